// ops.hip - the operations of a decoder layer besides Linear, for gfx950.
//
// Each kernel follows the arithmetic of the reference's CPU backend
// (src/infer/mormot.ai.infer.backend.cpu.pas) step by step - double sums
// where the CPU sums in double, single roundings where it rounds - so that a
// forward pass on the device gives the CPU's logits up to the order of
// double sums. Sums across lanes run as wave/block reductions.
#include "common.h"
#include "route.h"

namespace ihip {

// ------------------------------------------------------ activation quantizers
// xq row layout: int8 codes [in], then one float scale per 32-value group
// (the fp16 scale of a Q8_0 block as float, or the Q8_K super-block d repeated
// over its 8 groups). bad: set to 1 + the row when a value is not finite.
struct QuantArgs {
  const float* x;
  uint8_t* xq;
  int* bad;
  int32_t rows, in;
};

// InferQuantizeRowQ8_0 (backend.cpu.pas:634-689, ties to even): one lane per
// 32-value block
extern "C" __global__ __launch_bounds__(256) void quantize_q8_0(QuantArgs a)
{
  int G = a.in >> 5;
  int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int row = blockIdx.y;
  if (gi >= G) return;
  const float4* xp = (const float4*)(a.x + (int64_t)row * a.in + gi * 32);
  float v[32];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float4 t = xp[k];
    v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
  }
  float amax = 0.f;
  bool nonfinite = false;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    nonfinite |= (float_bits(v[j]) & 0x7f800000u) == 0x7f800000u;
    float m = fabsf(v[j]);
    if (m > amax) amax = m;
  }
  uint8_t* row_q = a.xq + (int64_t)row * ((int64_t)a.in + 4 * (int64_t)G);
  float* scales = (float*)(row_q + a.in);
  if (nonfinite && a.bad) a.bad[0] = 1 + row;
  float d = amax / 127.0f;
  uint16_t h = float_to_half(d);
  uint32_t q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (!(d < 2.9387359e-39f)) {
    float id = 1.0f / d;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      float t = v[j] * id;
      int c = (int)__builtin_rintf(t);
      q[j >> 2] |= ((uint32_t)c & 255u) << (8 * (j & 3));
    }
  }
  uint4* qp = (uint4*)(row_q + gi * 32);
  qp[0] = make_uint4(q[0], q[1], q[2], q[3]);
  qp[1] = make_uint4(q[4], q[5], q[6], q[7]);
  scales[gi] = half_to_float(h);
}

// InferQuantizeRowQ8_K (backend.cpu.pas:758-819): one wave per 256-value
// block, lane l holds values 4l..4l+3; the signed value of the largest
// magnitude, the first one on a tie, sets the scale
extern "C" __global__ __launch_bounds__(256) void quantize_q8_k(QuantArgs a)
{
  int NB = a.in >> 8;
  int G = a.in >> 5;
  int lane = threadIdx.x & 63;
  int64_t b = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  int row = blockIdx.y;
  if (b >= NB) return;
  const float4 t = ((const float4*)(a.x + (int64_t)row * a.in + b * 256))[lane];
  float v[4] = {t.x, t.y, t.z, t.w};
  float amax = 0.f, m = 0.f;
  int idx = 0x7fffffff;
  bool nonfinite = false;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    nonfinite |= (float_bits(v[j]) & 0x7f800000u) == 0x7f800000u;
    float f = fabsf(v[j]);
    if (f > amax) {
      amax = f;
      m = v[j];
      idx = 4 * lane + j;
    }
  }
  first_max<1>(amax, m, idx);
  first_max<2>(amax, m, idx);
  first_max<4>(amax, m, idx);
  first_max<8>(amax, m, idx);
  first_max<16>(amax, m, idx);
  first_max<32>(amax, m, idx);
  if (__any(nonfinite) && lane == 0 && a.bad) a.bad[0] = 1 + row;
  uint8_t* row_q = a.xq + (int64_t)row * ((int64_t)a.in + 4 * (int64_t)G);
  float* scales = (float*)(row_q + a.in);
  uint32_t q = 0;
  float d = 0.f;
  if (!(amax < 3.7320437e-37f)) {
    float iscale = -127.0f / m;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float tt = iscale * v[j];
      int c = (int)__builtin_rintf(tt);
      if (c > 127) c = 127;
      q |= ((uint32_t)c & 255u) << (8 * j);
    }
    d = 1.0f / iscale;
  }
  ((uint32_t*)(row_q + b * 256))[lane] = q;
  if (lane < 8) scales[b * 8 + lane] = d;
}

// ------------------------------------------------------------------ norms
// double sum over a block of 256 threads
__device__ double block_sum_d(double v, double* sh)
{
  v = wave_sum(v, 64);
  int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  double s = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
  return s;
}

struct NormArgs {
  float* x;        // rmsnorm: input; addnorm: residual, updated in place
  const float* t;  // addnorm: the added row, else null
  const float* w;
  float* y;
  double eps;
  int32_t rows, cols;
  // the MoE output of the row as its k expert rows cd [rows * k, cols] and
  // weights cw [rows * k], summed here in slot (= id) order (moecombine) and
  // added like t; null: t as given
  const float* cd;
  const float* cw;
  int32_t k, pad;
};

// TInferCpuBackend.RmsNorm (backend.cpu.pas:1769-1795): the sum of squares in
// double, inv = 1 / sqrt(mean + eps) in double, x * inv rounded to single
// before the weight; with t: x += t first (addnorm, ops.cu:135-150); with
// cd: x += the expert rows weighted in slot order, each step single-rounded
// as TDecoderModel.Experts adds them (decoder.pas:3140-3148)
// One block of 1024 per row; a thread keeps its NV columns c = t + 1024 i in
// registers and issues all their loads (and those of the k expert rows)
// before the first sum, so a row costs one memory round trip.
#define NORM_NV 4
extern "C" __global__ __launch_bounds__(1024) void rmsnorm(NormArgs a)
{
  __shared__ double sh[16];
  const int64_t base = (int64_t)blockIdx.x * a.cols;
  const int t = threadIdx.x;
  // a row of up to NORM_NV * 1024 columns stays in registers with its norm
  // weights, loaded with it: the output needs no second read
  const bool one = a.cols <= NORM_NV * 1024;
  float keep[NORM_NV], wv[NORM_NV];
  double s = 0;
  for (int c0 = 0; c0 < a.cols; c0 += NORM_NV * 1024) {
    float v[NORM_NV], add[NORM_NV];
#pragma unroll
    for (int i = 0; i < NORM_NV; i++) {
      int c = c0 + t + 1024 * i;
      v[i] = c < a.cols ? a.x[base + c] : 0.f;
      wv[i] = (one && c < a.cols) ? a.w[c] : 0.f;
      add[i] = 0.f;
    }
    if (a.cd) {
      float cwv[16];
      float cdv[16][NORM_NV];
#pragma unroll
      for (int j = 0; j < 16; j++) {
        int64_t sl = (int64_t)blockIdx.x * a.k + j;
        cwv[j] = j < a.k ? a.cw[sl] : 0.f;
#pragma unroll
        for (int i = 0; i < NORM_NV; i++) {
          int c = c0 + t + 1024 * i;
          cdv[j][i] = (j < a.k && c < a.cols) ? a.cd[sl * a.cols + c] : 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < 16; j++)
        if (j < a.k)
#pragma unroll
          for (int i = 0; i < NORM_NV; i++) {
            float p = cwv[j] * cdv[j][i];
            add[i] = add[i] + p;
          }
    } else if (a.t) {
#pragma unroll
      for (int i = 0; i < NORM_NV; i++) {
        int c = c0 + t + 1024 * i;
        add[i] = c < a.cols ? a.t[base + c] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < NORM_NV; i++) {
      int c = c0 + t + 1024 * i;
      keep[i] = 0.f;
      if (c < a.cols) {
        float x = v[i];
        if (a.cd || a.t) {
          x = x + add[i];
          a.x[base + c] = x;
        }
        keep[i] = x;
        double d = x;
        s = s + d * d;
      }
    }
  }
  s = wave_sum(s, 64);
  if ((t & 63) == 0) sh[t >> 6] = s;
  __syncthreads();
  s = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
  const double inv = 1.0 / sqrt(s / (double)a.cols + a.eps);
  if (one) {
#pragma unroll
    for (int i = 0; i < NORM_NV; i++) {
      int c = t + 1024 * i;
      if (c < a.cols) a.y[base + c] = wv[i] * (float)((double)keep[i] * inv);
    }
  } else {
    for (int c = t; c < a.cols; c += 1024) {
      float n = (float)((double)a.x[base + c] * inv);
      a.y[base + c] = a.w[c] * n;
    }
  }
}

// ------------------------------------------------ a block's output tail
// The row-wise steps between a block's output t and the next GEMV, in one
// launch (one block of 1024 per row, 4 columns a thread, cols <= 4096), each
// with the arithmetic of its own kernel (rmsnorm's sum order, so the bits of
// the separate launches):
//   t := norm(t) * dn_w                          (Gemma's dense output norm)
//   t := t + norm(sum_j ew_j * ed_j) * moe_w     (the experts beside it:
//                                                 moecombine, norm, add;
//                                                 ew null: weights 1, the
//                                                 rows summed already)
//   t := norm(t) * out_w                         (the block's output norm)
//   x := (x + t) * scalar[0]                     (residual, layer scalar)
//   h := norm(x) * nw                            (the next input norm)
// each step skipped when its operand is null (decoder.pas:2697-2702,
// 3057-3091, 3320-3336).
struct TailArgs {
  float* x;
  const float* t;
  const float* dn_w;
  const float* ed;
  const float* ew;
  const float* moe_w;
  const float* out_w;
  const float* scalar;
  const float* nw;
  float* h;
  double eps;
  int32_t rows, cols, k, pad;
};

// rmsnorm's arithmetic over a row held 4 columns a thread (v[i] = column
// t + 1024 i, 0 past the row): v := w * (float)(v * inv)
__device__ __forceinline__ void tail_norm(float (&v)[NORM_NV], const float (&w)[NORM_NV], int cols,
                                          double eps, double* sh)
{
  const int t = threadIdx.x;
  double s = 0;
#pragma unroll
  for (int i = 0; i < NORM_NV; i++)
    if (t + 1024 * i < cols) {
      const double d = v[i];
      s = s + d * d;
    }
  s = wave_sum(s, 64);
  __syncthreads();  // the previous norm's readers are done with sh
  if ((t & 63) == 0) sh[t >> 6] = s;
  __syncthreads();
  s = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
  const double inv = 1.0 / sqrt(s / (double)cols + eps);
#pragma unroll
  for (int i = 0; i < NORM_NV; i++) v[i] = w[i] * (float)((double)v[i] * inv);
}

extern "C" __global__ __launch_bounds__(1024) void row_tail(TailArgs a)
{
  __shared__ double sh[16];
  const int64_t base = (int64_t)blockIdx.x * a.cols;
  const int t = threadIdx.x;
  float tv[NORM_NV], xv[NORM_NV], wd[NORM_NV], wm[NORM_NV], wo[NORM_NV], wn[NORM_NV];
  float md[16][NORM_NV], mw[16];
  // every load first: the rows, the expert rows and their weights, the norms
#pragma unroll
  for (int i = 0; i < NORM_NV; i++) {
    const int c = t + 1024 * i;
    const bool in = c < a.cols;
    const int cc = in ? c : 0;
    tv[i] = in ? a.t[base + cc] : 0.f;
    xv[i] = in ? a.x[base + cc] : 0.f;
    wd[i] = a.dn_w ? a.dn_w[cc] : 0.f;
    wm[i] = a.moe_w ? a.moe_w[cc] : 0.f;
    wo[i] = a.out_w ? a.out_w[cc] : 0.f;
    wn[i] = a.nw[cc];
  }
  if (a.ed) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int64_t sl = (int64_t)blockIdx.x * a.k + min(j, a.k - 1);
      mw[j] = j < a.k ? (a.ew ? a.ew[sl] : 1.f) : 0.f;
#pragma unroll
      for (int i = 0; i < NORM_NV; i++) {
        const int c = t + 1024 * i;
        md[j][i] = (j < a.k && c < a.cols) ? a.ed[sl * a.cols + c] : 0.f;
      }
    }
  }
  if (a.dn_w) tail_norm(tv, wd, a.cols, a.eps, sh);
  if (a.ed) {
    // moecombine: the weighted expert rows in slot order, from 0
    float mv[NORM_NV];
#pragma unroll
    for (int i = 0; i < NORM_NV; i++) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j++)
        if (j < a.k) {
          const float p = mw[j] * md[j][i];
          acc = acc + p;
        }
      mv[i] = acc;
    }
    tail_norm(mv, wm, a.cols, a.eps, sh);
#pragma unroll
    for (int i = 0; i < NORM_NV; i++) tv[i] = tv[i] + mv[i];
  }
  if (a.out_w) tail_norm(tv, wo, a.cols, a.eps, sh);
  const float sc = a.scalar ? a.scalar[0] : 1.f;
#pragma unroll
  for (int i = 0; i < NORM_NV; i++) {
    float x = xv[i] + tv[i];
    if (a.scalar) x = x * sc;
    xv[i] = x;
    const int c = t + 1024 * i;
    if (c < a.cols) a.x[base + c] = x;
  }
  tail_norm(xv, wn, a.cols, a.eps, sh);
#pragma unroll
  for (int i = 0; i < NORM_NV; i++) {
    const int c = t + 1024 * i;
    if (c < a.cols) a.h[base + c] = xv[i];
  }
}

struct EltArgs {
  float* x;
  const float* t;
  int64_t n;
  float alpha, limit;
};

// x := x + t (TInferBackend.Add)
extern "C" __global__ __launch_bounds__(256) void add(EltArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.n) a.x[i] = a.x[i] + a.t[i];
}

// TInferCpuBackend.SwiGlu (backend.cpu.pas:1797-1834): x = gate, t = up
extern "C" __global__ __launch_bounds__(256) void swiglu(EltArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  if (a.limit > 0) {
    float g = a.x[i], u = a.t[i];
    if (g > a.limit) g = a.limit;
    if (u > a.limit) u = a.limit;
    else if (u < -a.limit) u = -a.limit;
    float b = g * a.alpha;
    double d = b;
    b = (float)(1.0 / (1.0 + exp(-d)));
    b = g * b;
    u = u + 1.0f;
    a.x[i] = u * b;
  } else {
    double d = a.x[i];
    float b = (float)(d / (1.0 + exp(-d)));
    a.x[i] = b * a.t[i];
  }
}

// TInferCpuBackend.GeluTanhGlu (backend.cpu.pas:1836-1860): x = gate, t = up
// (geglu_value)
extern "C" __global__ __launch_bounds__(256) void geglu(EltArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  a.x[i] = geglu_value(a.x[i], a.t[i]);
}

// x := x * t[0] (Gemma's layer scalar, decoder.pas:3330-3336), or x * alpha
// with t null (the embedding scale, :3305-3309)
extern "C" __global__ __launch_bounds__(256) void mul_scalar(EltArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const float s = a.t ? a.t[0] : a.alpha;
  a.x[i] = a.x[i] * s;
}

struct SoftcapArgs {
  float* x;
  int64_t n;
  double cap;
};

// InferSoftcap (decoder.pas:1293-1312): tanh(x / c) * c, each step single
extern "C" __global__ __launch_bounds__(256) void softcap(SoftcapArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const float v = (float)(a.x[i] / a.cap);
  const double d = v;
  float t;
  if (d > 20) t = 1;
  else if (d < -20) t = -1;
  else t = (float)(1 - 2 / (exp(2 * d) + 1));
  a.x[i] = (float)(t * a.cap);
}

// ------------------------------------------------------------------ qkrope
struct RopeArgs {
  float* q;
  const float* k;
  const float* v;
  const float* qn;  // [hd] or null: no per-head norm
  const float* kn;
  const float* cs;  // [rows, hd/2] cos, then [rows, hd/2] sin; null: no rotary
                    // positions (a NoPE layer, TDecoderLayerSpec.NoRope)
  void* kc;         // cache [*, kvh * hd] float or half
  void* vc;
  const int* pastp;  // device position of row 0 (graph replay), or null: past
  double eps;
  int32_t rows, heads, kvh, hd, past, f16;
  int32_t rot;       // the rotating values of a head from its start (0: all)
  int32_t vnorm;     // 1: every V head RMS-normed without weight (ValueNorm)
};

// per (head: the q heads, then the kv heads; row): the Q/K head RMSNorm of
// decoder.pas:2668-2673, rotate_half RoPE in double over the first rot
// values (backend.cpu.pas:1862-1888; cs holds [rows, rot / 2] cos, then
// sin), K and V stored into the cache at past + row (decoder.pas:
// 2688-2691); one wave per head
extern "C" __global__ __launch_bounds__(64) void qkrope(RopeArgs a)
{
  // every operand loaded first (heads up to 512: 8 values and 4 rotary
  // pairs a thread), then the arithmetic: one memory round trip
  constexpr int NV = 8, NR = 4;
  __shared__ float nv[512];
  int hh = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  // (a NoPE layer: no rotating part, every value normed and stored as it is)
  int d = a.hd, half = a.cs ? (a.rot > 0 ? a.rot : d) >> 1 : 0;
  const int past = a.pastp ? *a.pastp : a.past;
  bool isq = hh < a.heads;
  int h = isq ? hh : hh - a.heads;
  int64_t src = isq ? ((int64_t)r * a.heads + h) * d : ((int64_t)r * a.kvh + h) * d;
  const float* in = isq ? a.q + src : a.k + src;
  const float* nw = isq ? a.qn : a.kn;
  const float* cr = a.cs ? a.cs + (int64_t)r * half : nullptr;
  const float* sr = a.cs ? a.cs + (int64_t)a.rows * half + (int64_t)r * half : nullptr;
  float xin[NV], wv[NV], vin[NV], cv[NR], sv[NR];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int cc = min(t + 64 * i, d - 1);
    xin[i] = in[cc];
    wv[i] = nw ? nw[cc] : 1.f;
    vin[i] = isq ? 0.f : a.v[src + cc];
  }
#pragma unroll
  for (int j = 0; j < NR; j++) {
    const int ii = min(t + 64 * j, max(half - 1, 0));
    cv[j] = a.cs ? cr[ii] : 1.f;
    sv[j] = a.cs ? sr[ii] : 0.f;
  }
  if (nw) {
    double s = 0;
#pragma unroll
    for (int i = 0; i < NV; i++)
      if (t + 64 * i < d) {
        double x = xin[i];
        s = s + x * x;
      }
    s = wave_sum(s, 64);
    double inv = 1.0 / sqrt(s / (double)d + a.eps);
#pragma unroll
    for (int i = 0; i < NV; i++)
      if (t + 64 * i < d) {
        float n = (float)((double)xin[i] * inv);
        nv[t + 64 * i] = wv[i] * n;
      }
  } else {
#pragma unroll
    for (int i = 0; i < NV; i++)
      if (t + 64 * i < d) nv[t + 64 * i] = xin[i];
  }
  __syncthreads();
  int64_t kvw = (int64_t)a.kvh * d;
  int64_t dst = ((int64_t)past + r) * kvw + (int64_t)h * d;
#pragma unroll
  for (int j = 0; j < NR; j++) {
    const int i = t + 64 * j;
    if (i >= half) break;
    double x0 = nv[i], x1 = nv[i + half], c = cv[j], s = sv[j];
    float o0 = (float)(x0 * c - x1 * s);
    float o1 = (float)(x1 * c + x0 * s);
    if (isq) {
      a.q[src + i] = o0;
      a.q[src + i + half] = o1;
    } else if (a.f16) {
      ((uint16_t*)a.kc)[dst + i] = float_to_half(o0);
      ((uint16_t*)a.kc)[dst + i + half] = float_to_half(o1);
    } else {
      ((float*)a.kc)[dst + i] = o0;
      ((float*)a.kc)[dst + i + half] = o1;
    }
  }
  // the values beyond the rotating part: normed, not rotated
  for (int c = 2 * half + t; c < d; c += 64) {
    float o = nv[c];
    if (isq) a.q[src + c] = o;
    else if (a.f16) ((uint16_t*)a.kc)[dst + c] = float_to_half(o);
    else ((float*)a.kc)[dst + c] = o;
  }
  if (!isq) {
    // ValueNorm (decoder.pas:2674-2676): the RMSNorm of RmsNorm with unit
    // weights, so the normed value itself
    double inv = 1.0;
    if (a.vnorm) {
      double sv2 = 0;
#pragma unroll
      for (int i = 0; i < NV; i++)
        if (t + 64 * i < d) {
          double x = vin[i];
          sv2 = sv2 + x * x;
        }
      sv2 = wave_sum(sv2, 64);
      inv = 1.0 / sqrt(sv2 / (double)d + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c = t + 64 * i;
      if (c >= d) break;
      float vv = vin[i];
      if (a.vnorm) vv = 1.0f * (float)((double)vv * inv);
      if (a.f16) ((uint16_t*)a.vc)[dst + c] = float_to_half(vv);
      else ((float*)a.vc)[dst + c] = vv;
    }
  }
}

// --------------------------------------------------------------- attention
struct AttnArgs {
  const float* q;
  const void* kc;
  const void* vc;
  float* y;
  const float* sinks;
  const int* pastp;  // device position of row 0 (graph replay), or null: past
  double* part;      // [heads, rows, splits, hd + 2] partial sums, maxima, sums
  double scale;
  int32_t rows, heads, kvh, hd, past, window, f16, splits;
};

__device__ __forceinline__ double cache_at(const void* c, int64_t i, int f16)
{
  return f16 ? (double)half_to_float(((const uint16_t*)c)[i]) : (double)((const float*)c)[i];
}

// the head of block x of an attention launch over (heads, ...): consecutive
// heads - one KV group's query heads, which read the same key and value
// tiles - on one XCD. The workgroups of a launch go to the 8 XCDs in turn by
// block id (x first), each XCD with its own L2; with heads a multiple of 8,
// block x runs on XCD x % 8 whatever its y and z.
__device__ __forceinline__ int xcd_head(unsigned x, int heads)
{
  return (heads & 7) ? (int)x : (int)(x & 7) * (heads >> 3) + (int)(x >> 3);
}

// the keys of one (head, row) cut into `splits` ranges of at most ATT_CHUNK
// keys (flash-decoding): each block scores its range in double, then sums
// exp(score - range max) and the weighted values in double, and writes them
// with the range's maximum and sum to part; attention_merge adds the ranges
// (and the sink) as the CPU adds one softmax. Not the CPU's exact bits
// (CausalRows, backend.cpu.pas:1305-1354): f16 keys of heads that are a
// multiple of 16 are scored in another order of the double sum (two halves,
// four chains each), and every value is added by a fused multiply-add of the
// double weight p and the value (p * v is not exact in double, so one rounding
// where the CPU has two). Both differ from the CPU in the last bits of a
// double, far below the f32 rounding of the output (within 2 f32 ulp of the
// oracle in the tests). Every load of a
// range is issued before its first use: one thread per key reads the whole
// key row at once, and each lane of the value pass holds a dimension pair of
// all its keys, so a block waits for memory once per pass.
#define ATT_CHUNK 128
// NP: dimension pairs per lane in the value pass, 2 for heads up to 256, 4
// for heads up to 512 (Gemma 4's full layers)
template <bool F16, int NP = 2>
__device__ __forceinline__ void attention_part_t(const AttnArgs& a)
{
  __shared__ double qd[128 * NP];
  __shared__ double sc[ATT_CHUNK];
  __shared__ double red[8];
  __shared__ double accs[4][128 * NP];
  const int h = xcd_head(blockIdx.x, a.heads), r = blockIdx.y, s = blockIdx.z, t = threadIdx.x;
  const int d = a.hd;
  const int64_t kvw = (int64_t)a.kvh * d, qw = (int64_t)a.heads * d;
  const int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  const int total = past + r + 1;
  const int first = (a.window > 0 && total > a.window) ? total - a.window : 0;
  const int cnt = total - first;
  const int j0 = min(cnt, s * ATT_CHUNK), j1 = min(cnt, j0 + ATT_CHUNK);
  const int n = j1 - j0;
  double* out = a.part + (((int64_t)h * a.rows + r) * a.splits + s) * (d + 2);
  if (n <= 0) {  // an empty range: weight 0 in the merge
    if (t == 0) {
      out[d] = -1.0e308;
      out[d + 1] = 0.0;
    }
    return;
  }
  const float* q = a.q + (int64_t)r * qw + (int64_t)h * d;
  for (int i = t; i < d; i += 256) qd[i] = (double)q[i];
  __syncthreads();
  double m = -1.0e308;
  const int64_t base = (int64_t)(first + j0) * kvw + (int64_t)g * d;
  // f16 keys whose halves are whole 16-byte words: two threads a key, each half of the
  // dimensions in four interleaved fused multiply-add chains (q and k are
  // float values, so each product is exact in double and the fused add
  // rounds as the CPU's add; only the order of the double sum differs);
  // otherwise a thread a key in the CPU's order
  const bool paired = F16 && !(d & 15);
  if (paired) {
    const int kk = t >> 1, hh = t & 1;
    const int nw16 = d / 16;  // 16-byte words of half a key row
    double c4[4] = {0, 0, 0, 0};
    if (kk < n) {
      const uint4* p = (const uint4*)((const uint16_t*)a.kc + base + (int64_t)kk * kvw) + hh * nw16;
      for (int k0 = 0; k0 < nw16; k0 += 16) {
        uint4 u[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < nw16) u[k] = p[k0 + k];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < nw16) {
            const uint32_t wv[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const int i = hh * (d / 2) + 8 * (k0 + k) + 2 * j;
              c4[(2 * j) & 3] = __builtin_fma(qd[i], (double)half_to_float(wv[j] & 0xffffu), c4[(2 * j) & 3]);
              c4[(2 * j + 1) & 3] =
                  __builtin_fma(qd[i + 1], (double)half_to_float(wv[j] >> 16), c4[(2 * j + 1) & 3]);
            }
          }
      }
    }
    const double part = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    double acc = part + xpart<1>(part);  // the other half of the key
    acc = acc * a.scale;
    if (kk < n) {
      if (hh == 0) sc[kk] = acc;
      m = acc;
    }
  } else if (t < n) {
    const int64_t kb = base + (int64_t)t * kvw;
    double acc = 0;
    if (F16 && (d & 7)) {
      // a head that is no multiple of 8 (rows not 16-byte aligned): one by one
      for (int i = 0; i < d; i++) acc = acc + qd[i] * (double)half_to_float(((const uint16_t*)a.kc)[kb + i]);
    } else if (!F16 && (d & 3)) {
      for (int i = 0; i < d; i++) acc = acc + qd[i] * (double)((const float*)a.kc)[kb + i];
    } else if constexpr (F16) {
      const uint4* p = (const uint4*)((const uint16_t*)a.kc + kb);
      for (int k0 = 0; k0 < d / 8; k0 += 16) {
        uint4 u[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < d / 8) u[k] = p[k0 + k];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < d / 8) {
            uint32_t wv[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
              int i = 8 * (k0 + k) + 2 * j;
              acc = acc + qd[i] * (double)half_to_float(wv[j] & 0xffffu);
              acc = acc + qd[i + 1] * (double)half_to_float(wv[j] >> 16);
            }
          }
      }
    } else {
      const float4* p = (const float4*)((const float*)a.kc + kb);
      for (int k0 = 0; k0 < d / 4; k0 += 16) {
        float4 u[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < d / 4) u[k] = p[k0 + k];
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (k0 + k < d / 4) {
            int i = 4 * (k0 + k);
            acc = acc + qd[i] * (double)u[k].x;
            acc = acc + qd[i + 1] * (double)u[k].y;
            acc = acc + qd[i + 2] * (double)u[k].z;
            acc = acc + qd[i + 3] * (double)u[k].w;
          }
      }
    }
    acc = acc * a.scale;
    sc[t] = acc;
    m = acc;
  }
  m = wave_max(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
  double e = 0;
  if (t < n) {
    e = exp(sc[t] - m);
    sc[t] = e;
  }
  e = wave_sum(e, 64);
  __syncthreads();
  if ((t & 63) == 0) red[4 + (t >> 6)] = e;
  // the weighted values: a key takes a slot of lps lanes (hd / 2 rounded up
  // to a power of two, at most 64), each lane a dimension pair (up to NP of
  // them for hd > 128); lanes past the key's pairs hold zeros. The 4 waves
  // and the key slots of a wave split the range.
  const int lpk = d >> 1;                                      // dimension pairs of a key
  const int lps = lpk >= 64 ? 64 : 1 << (32 - __clz(lpk - 1));  // lanes per key slot
  const int kpw = 64 / lps;                                    // keys side by side in a wave
  const int w = t >> 6, l = t & 63;
  const int lane_key = l / lps, pair = l % lps;
  const int step = 4 * kpw;
  double a0[NP], a1[NP];  // the lane's dimension pairs pair, pair + 64, ..
#pragma unroll
  for (int c = 0; c < NP; c++) a0[c] = a1[c] = 0;
  int npair = 0;
#pragma unroll
  for (int c = 0; c < NP; c++)
    if (pair + 64 * c < lpk) npair = c + 1;
  constexpr int VB = (F16 ? 32 : 16) * 2 / NP;  // value loads in flight per lane
  for (int jb = w * kpw + lane_key; jb < n; jb += VB * step) {
    if constexpr (F16) {
      uint32_t v[VB][NP];
#pragma unroll
      for (int u = 0; u < VB; u++) {
        int j = jb + u * step;
#pragma unroll
        for (int c = 0; c < NP; c++)
          v[u][c] = (j < n && c < npair)
                        ? ((const uint32_t*)((const uint16_t*)a.vc + base + (int64_t)j * kvw))[pair + 64 * c]
                        : 0u;
      }
#pragma unroll
      for (int u = 0; u < VB; u++) {
        int j = jb + u * step;
        if (j < n) {
          double p = sc[j];
#pragma unroll
          for (int c = 0; c < NP; c++)
            if (c < npair) {
              a0[c] = __builtin_fma(p, (double)half_to_float(v[u][c] & 0xffffu), a0[c]);
              a1[c] = __builtin_fma(p, (double)half_to_float(v[u][c] >> 16), a1[c]);
            }
        }
      }
    } else {
      float2 v[VB][NP];
#pragma unroll
      for (int u = 0; u < VB; u++) {
        int j = jb + u * step;
#pragma unroll
        for (int c = 0; c < NP; c++)
          v[u][c] = (j < n && c < npair)
                        ? ((const float2*)((const float*)a.vc + base + (int64_t)j * kvw))[pair + 64 * c]
                        : make_float2(0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < VB; u++) {
        int j = jb + u * step;
        if (j < n) {
          double p = sc[j];
#pragma unroll
          for (int c = 0; c < NP; c++)
            if (c < npair) {
              a0[c] = __builtin_fma(p, (double)v[u][c].x, a0[c]);
              a1[c] = __builtin_fma(p, (double)v[u][c].y, a1[c]);
            }
        }
      }
    }
  }
  // the key slots of a wave, then the waves
  for (int o = lps; o < 64; o <<= 1)
#pragma unroll
    for (int c = 0; c < NP; c++) {
      a0[c] += __shfl_xor(a0[c], o);
      a1[c] += __shfl_xor(a1[c], o);
    }
  if (lane_key == 0)
#pragma unroll
    for (int c = 0; c < NP; c++)
      if (c < npair) {
        accs[w][2 * (pair + 64 * c)] = a0[c];
        accs[w][2 * (pair + 64 * c) + 1] = a1[c];
      }
  __syncthreads();
  for (int i = t; i < d; i += 256) out[i] = (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]);
  if (t == 0) {
    out[d] = m;
    out[d + 1] = (red[4] + red[5]) + (red[6] + red[7]);
  }
}

// The ranges of ATTR rows at once (prompt chunks, head_dim HD = 64 or 128):
// one block per (head, tile of ATTR consecutive rows, range s). Row r's
// range s is its keys first_r + s * ATT_CHUNK .. (its own window start and
// causal end); the tile's rows together need at most ATT_CHUNK + ATTR - 1
// keys, loaded once for all of them (attention_part loads them per row).
// The arithmetic of a row is attention_part's: every score the CPU's
// sequential double dot product, exp(score - range max) and the weighted
// values in double, here summed in key order per row.
constexpr int ATTR = 8;
constexpr int ATTK = ATT_CHUNK + ATTR - 1;  // keys of a tile's range
template <bool F16, int HD>
__device__ __forceinline__ void attention_rows_t(const AttnArgs& a)
{
  __shared__ double qd[ATTR][HD];
  __shared__ double sc[ATTR][ATTK + 1];
  __shared__ double stat[ATTR][2];  // a row's range maximum and sum
  const int h = xcd_head(blockIdx.x, a.heads), r0 = blockIdx.y * ATTR, s = blockIdx.z, t = threadIdx.x;
  constexpr int d = HD;
  const int64_t kvw = (int64_t)a.kvh * d, qw = (int64_t)a.heads * d;
  const int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  // row r (tile row, r0 + r < rows): absolute keys [k0[r], k1[r]) of range s
  auto range = [&](int r, int& k0, int& k1) {
    const int total = past + r0 + r + 1;
    const int first = (a.window > 0 && total > a.window) ? total - a.window : 0;
    const int cnt = total - first;
    const int j0 = min(cnt, s * ATT_CHUNK), j1 = min(cnt, j0 + ATT_CHUNK);
    k0 = first + j0;
    k1 = first + j1;
    if (r0 + r >= a.rows) k0 = k1 = 0;
  };
  int kb, dummy;
  range(0, kb, dummy);  // the tile's first key (row 0 starts earliest)
  for (int i = t; i < ATTR * d; i += 256) {
    const int r = i / d, c = i % d;
    qd[r][c] = r0 + r < a.rows ? (double)a.q[(int64_t)(r0 + r) * qw + (int64_t)h * d + c] : 0.0;
  }
  __syncthreads();
  // ---- scores: a thread per key of the tile, the rows' dots in key-row order
  if (t < ATTK) {
    const int key = kb + t;
    bool in[ATTR];
    bool any = false;
#pragma unroll
    for (int r = 0; r < ATTR; r++) {
      int k0, k1;
      range(r, k0, k1);
      in[r] = key >= k0 && key < k1;
      any |= in[r];
    }
    double acc[ATTR];
#pragma unroll
    for (int r = 0; r < ATTR; r++) acc[r] = 0.0;
    if (any) {
      const int64_t kr = (int64_t)key * kvw + (int64_t)g * d;
      if constexpr (F16) {
        const uint4* p = (const uint4*)((const uint16_t*)a.kc + kr);
        uint4 u[d / 8];
#pragma unroll
        for (int k = 0; k < d / 8; k++) u[k] = p[k];
#pragma unroll
        for (int k = 0; k < d / 8; k++) {
          const uint32_t wv[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int i = 8 * k + 2 * j;
            const double k0v = (double)half_to_float(wv[j] & 0xffffu), k1v = (double)half_to_float(wv[j] >> 16);
            // q * k is exact in double: a fused multiply-add rounds as the
            // CPU's multiply-then-add
#pragma unroll
            for (int r = 0; r < ATTR; r++) {
              acc[r] = __builtin_fma(qd[r][i], k0v, acc[r]);
              acc[r] = __builtin_fma(qd[r][i + 1], k1v, acc[r]);
            }
          }
        }
      } else {
        const float4* p = (const float4*)((const float*)a.kc + kr);
#pragma unroll 4
        for (int k = 0; k < d / 4; k++) {
          const float4 u = p[k];
          const double kv[4] = {(double)u.x, (double)u.y, (double)u.z, (double)u.w};
#pragma unroll
          for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < ATTR; r++) acc[r] = __builtin_fma(qd[r][4 * k + j], kv[j], acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < ATTR; r++) sc[r][t] = in[r] ? acc[r] * a.scale : -1.0e308;
  }
  __syncthreads();
  // ---- per row: the range maximum, the weights exp(score - max), their sum
  // (wave w takes rows 2w and 2w + 1)
  const int w = t >> 6, l = t & 63;
#pragma unroll
  for (int rr = 0; rr < 2; rr++) {
    const int r = 2 * w + rr;
    double m = -1.0e308;
    for (int j = l; j < ATTK; j += 64) m = fmax(m, sc[r][j]);
    m = wave_max(m);
    double e = 0;
    for (int j = l; j < ATTK; j += 64) {
      const double x = sc[r][j];
      const double p = x > -1.0e308 ? exp(x - m) : 0.0;
      sc[r][j] = p;
      e += p;
    }
    e = wave_sum(e, 64);
    if (l == 0) {
      stat[r][0] = m;
      stat[r][1] = e;
    }
  }
  __syncthreads();
  // ---- the weighted values: wave w, rows 2w and 2w + 1; a lane holds a
  // dimension pair (HD 64: lanes 32.. take every other key, added at the end)
  constexpr int LPK = HD / 2;               // lanes per key
  constexpr int KPW = 64 / LPK;             // keys side by side in a wave
  const int pair = l % LPK, ks = l / LPK;
  double a00 = 0, a01 = 0, a10 = 0, a11 = 0;  // [row][dim]
  const int64_t vb = (int64_t)kb * kvw + (int64_t)g * d + 2 * pair;
  constexpr int VB = 16;  // value loads in flight per lane
  for (int j0 = ks; j0 < ATTK; j0 += VB * KPW) {
    float2 v[VB];
#pragma unroll
    for (int u = 0; u < VB; u++) {
      const int j = min(j0 + u * KPW, ATTK - 1);
      // a key past the cache's end reads the tile's first key (weight 0)
      const int64_t e = (kb + j < (int64_t)past + a.rows) ? vb + (int64_t)j * kvw : vb;
      if constexpr (F16) {
        const uint32_t x = *(const uint32_t*)((const uint16_t*)a.vc + e);
        v[u] = make_float2(half_to_float(x & 0xffffu), half_to_float(x >> 16));
      } else {
        v[u] = *(const float2*)((const float*)a.vc + e);
      }
    }
#pragma unroll
    for (int u = 0; u < VB; u++) {
      const int j = j0 + u * KPW;
      if (j < ATTK) {
        const double p0 = sc[2 * w][j], p1 = sc[2 * w + 1][j];
        a00 = a00 + p0 * (double)v[u].x;
        a01 = a01 + p0 * (double)v[u].y;
        a10 = a10 + p1 * (double)v[u].x;
        a11 = a11 + p1 * (double)v[u].y;
      }
    }
  }
  if constexpr (KPW == 2) {
    a00 = a00 + xpart<32>(a00);
    a01 = a01 + xpart<32>(a01);
    a10 = a10 + xpart<32>(a10);
    a11 = a11 + xpart<32>(a11);
  }
#pragma unroll
  for (int rr = 0; rr < 2; rr++) {
    const int r = 2 * w + rr;
    if (r0 + r >= a.rows) continue;
    double* out = a.part + (((int64_t)h * a.rows + r0 + r) * a.splits + s) * (d + 2);
    if (ks == 0) {
      out[2 * pair] = rr ? a10 : a00;
      out[2 * pair + 1] = rr ? a11 : a01;
    }
    if (l == 0) {
      // an empty range: weight 0 in the merge
      const bool empty = !(stat[r][1] > 0.0);
      out[d] = empty ? -1.0e308 : stat[r][0];
      out[d + 1] = empty ? 0.0 : stat[r][1];
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void attention_rows_f16_64(AttnArgs a)
{
  attention_rows_t<true, 64>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_rows_f16_128(AttnArgs a)
{
  attention_rows_t<true, 128>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_rows_f32_64(AttnArgs a)
{
  attention_rows_t<false, 64>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_rows_f32_128(AttnArgs a)
{
  attention_rows_t<false, 128>(a);
}

// The ranges of ATTM rows at once on the f64 matrix cores (prompt chunks,
// head_dim HD = 64 or 128): one block per (head, tile of ATTM = 16
// consecutive rows, range s), the rows' ranges as attention_rows forms them
// (a tile's keys span at most ATT_CHUNK + 15). Scores Q K^T and the weighted
// values P V are v_mfma_f64_16x16x4f64 products: q (float), the cached keys
// and values (half or float) and the weights are exact as doubles, every
// product is exact and the sums run in double - only their order differs
// from the CPU's sequential dot (CausalRows, backend.cpu.pas:1305-1354), a
// difference of the order of 1e-16 relative before the result is rounded
// to single. Per MFMA, lane l holds A[l % 16][l / 16] and B[l / 16][l % 16];
// D[l / 16 + 4 v][l % 16] comes back in its register v. The k index of a
// lane group (l / 16) runs over a contiguous quarter of the dimensions (the
// scores) or of the tile's keys (the values), so each lane reads its own
// contiguous part of a row: the sum is over the same terms, permuted.
constexpr int ATTM = 16;
constexpr int ATTMK = ATT_CHUNK + ATTM;  // keys of a tile's range, padded to 16
typedef double dbl4 __attribute__((ext_vector_type(4)));

template <bool F16, int HD>
__device__ __forceinline__ void attention_mfma_t(const AttnArgs& a)
{
  __shared__ double sc[ATTM][ATTMK + 1];  // scores, then weights (row, tile key)
  __shared__ double stat[ATTM][2];
  __shared__ int rk[ATTM][2];             // a row's keys [k0, k1) (absolute)
  const int h = xcd_head(blockIdx.x, a.heads), r0 = blockIdx.y * ATTM, s = blockIdx.z;
  const int t = threadIdx.x, w = t >> 6, l = t & 63, lq = l >> 4, lc = l & 15;
  constexpr int d = HD;
  const int64_t kvw = (int64_t)a.kvh * d, qw = (int64_t)a.heads * d;
  const int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  if (t < ATTM) {
    const int r = t;
    const int total = past + r0 + r + 1;
    const int first = (a.window > 0 && total > a.window) ? total - a.window : 0;
    const int cnt = total - first;
    const int j0 = min(cnt, s * ATT_CHUNK), j1 = min(cnt, j0 + ATT_CHUNK);
    int k0 = first + j0, k1 = first + j1;
    if (r0 + r >= a.rows || k0 >= k1) k0 = k1 = -1;  // no key of this range
    rk[r][0] = k0;
    rk[r][1] = k1;
  }
  __syncthreads();
  // the tile's keys [kb, ke): from the first row with keys to the last
  int kb = 0x7fffffff, ke = -1;
#pragma unroll
  for (int r = 0; r < ATTM; r++)
    if (rk[r][0] >= 0) {
      kb = min(kb, rk[r][0]);
      ke = max(ke, rk[r][1]);
    }
  const int nblk = ke > kb ? (ke - kb + 15) >> 4 : 0;  // blocks of 16 keys (<= 9)
  if (nblk > 0) {
    // ---- scores: wave w takes key blocks w, w + 4, w + 8; lane group lq
    // the dimensions [lq * d / 4, (lq + 1) * d / 4)
    constexpr int DQ = d / 4;  // k steps = a lane's dimensions
    const int qr = min(r0 + lc, a.rows - 1);
    double qa[DQ];
    {
      const float4* qp = (const float4*)(a.q + (int64_t)qr * qw + (int64_t)h * d + lq * DQ);
#pragma unroll
      for (int i = 0; i < DQ / 4; i++) {
        const float4 u = qp[i];
        qa[4 * i] = u.x;
        qa[4 * i + 1] = u.y;
        qa[4 * i + 2] = u.z;
        qa[4 * i + 3] = u.w;
      }
    }
    for (int kbk = w; kbk < nblk; kbk += 4) {
      const int key = min(kb + 16 * kbk + lc, ke - 1);
      const int64_t kr = (int64_t)key * kvw + (int64_t)g * d + lq * DQ;
      constexpr int NW = F16 ? DQ / 8 : DQ / 4;  // 16-byte words of a lane's part
      uint4 u[NW];
      if constexpr (F16) {
        const uint4* p = (const uint4*)((const uint16_t*)a.kc + kr);
#pragma unroll
        for (int i = 0; i < NW; i++) u[i] = p[i];
      } else {
        const uint4* p = (const uint4*)((const float*)a.kc + kr);
#pragma unroll
        for (int i = 0; i < NW; i++) u[i] = p[i];
      }
      dbl4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int i = 0; i < NW; i++) {
        const uint32_t wv[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if constexpr (F16) {
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[8 * i + 2 * j], (double)half_to_float(wv[j] & 0xffffu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[8 * i + 2 * j + 1], (double)half_to_float(wv[j] >> 16), acc, 0, 0, 0);
          } else {
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[4 * i + j], (double)bits_float(wv[j]), acc, 0, 0, 0);
          }
        }
      }
      // D[row][key]: row lq + 4 v, key column lc of this block
      const int kk = 16 * kbk + lc, kabs = kb + kk;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int r = lq + 4 * v;
        const bool in = kabs >= rk[r][0] && kabs < rk[r][1];
        sc[r][kk] = in ? acc[v] * a.scale : -1.0e308;
      }
    }
  }
  __syncthreads();
  const int nk = 16 * nblk;
  // ---- per row: the range maximum, the weights exp(score - max), their sum
  // (wave w takes rows 4w .. 4w + 3)
#pragma unroll
  for (int rr = 0; rr < 4; rr++) {
    const int r = 4 * w + rr;
    double m = -1.0e308;
    for (int j = l; j < nk; j += 64) m = fmax(m, sc[r][j]);
    m = wave_max(m);
    double e = 0;
    for (int j = l; j < nk; j += 64) {
      const double x = sc[r][j];
      const double p = x > -1.0e308 ? exp(x - m) : 0.0;
      sc[r][j] = p;
      e += p;
    }
    e = wave_sum(e, 64);
    if (l == 0) {
      stat[r][0] = m;
      stat[r][1] = e;
    }
  }
  __syncthreads();
  // ---- the weighted values: wave w the dimensions [w * d / 4, (w + 1) *
  // d / 4) as NT tiles of 16 (HD 128: the even and the odd dimensions of the
  // wave's 32); lane group lq the tile keys [lq * S, (lq + 1) * S)
  constexpr int NT = d / 64;
  const int S = nk >> 2;  // k steps (nk is a multiple of 16)
  dbl4 o[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) o[n] = dbl4{0.0, 0.0, 0.0, 0.0};
  if (nblk > 0) {
    const int dim0 = w * (d / 4) + NT * lc;  // this lane's column dimension(s)
    const int64_t vb = (int64_t)g * d + dim0;
    constexpr int VU = 12;  // value loads in flight per lane
    for (int t0 = 0; t0 < S; t0 += VU) {
      float vv[VU][NT];
#pragma unroll
      for (int u = 0; u < VU; u++) {
        const int key = min(kb + lq * S + min(t0 + u, S - 1), ke - 1);
        const int64_t e = (int64_t)key * kvw + vb;
        if constexpr (F16) {
          if constexpr (NT == 2) {
            const uint32_t x = *(const uint32_t*)((const uint16_t*)a.vc + e);
            vv[u][0] = half_to_float(x & 0xffffu);
            vv[u][1] = half_to_float(x >> 16);
          } else {
            vv[u][0] = half_to_float(((const uint16_t*)a.vc)[e]);
          }
        } else {
          if constexpr (NT == 2) {
            const float2 x = *(const float2*)((const float*)a.vc + e);
            vv[u][0] = x.x;
            vv[u][1] = x.y;
          } else {
            vv[u][0] = ((const float*)a.vc)[e];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < VU; u++) {
        if (t0 + u < S) {
          const double p = sc[lc][lq * S + t0 + u];
#pragma unroll
          for (int n = 0; n < NT; n++)
            o[n] = __builtin_amdgcn_mfma_f64_16x16x4f64(p, (double)vv[u][n], o[n], 0, 0, 0);
        }
      }
    }
  }
  // ---- the partial results: row lq + 4 v, dimension(s) dim0 + n
  const int dim0 = w * (d / 4) + NT * lc;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int r = lq + 4 * v;
    if (r0 + r >= a.rows) continue;
    double* out = a.part + (((int64_t)h * a.rows + r0 + r) * a.splits + s) * (d + 2);
#pragma unroll
    for (int n = 0; n < NT; n++) out[dim0 + n] = o[n][v];
  }
  if (t < ATTM && r0 + t < a.rows) {
    double* out = a.part + (((int64_t)h * a.rows + r0 + t) * a.splits + s) * (d + 2);
    const bool empty = !(stat[t][1] > 0.0);
    out[d] = empty ? -1.0e308 : stat[t][0];
    out[d + 1] = empty ? 0.0 : stat[t][1];
  }
}

extern "C" __global__ __launch_bounds__(256) void attention_mfma_f16_64(AttnArgs a)
{
  attention_mfma_t<true, 64>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_mfma_f16_128(AttnArgs a)
{
  attention_mfma_t<true, 128>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_mfma_f32_64(AttnArgs a)
{
  attention_mfma_t<false, 64>(a);
}
extern "C" __global__ __launch_bounds__(256) void attention_mfma_f32_128(AttnArgs a)
{
  attention_mfma_t<false, 128>(a);
}

extern "C" __global__ __launch_bounds__(256) void attention_part_f16(AttnArgs a)
{
  attention_part_t<true>(a);
}

extern "C" __global__ __launch_bounds__(256) void attention_part_f32(AttnArgs a)
{
  attention_part_t<false>(a);
}

// heads of 257..512 values (Gemma 4's full layers)
extern "C" __global__ __launch_bounds__(256) void attention_part_f16_512(AttnArgs a)
{
  attention_part_t<true, 4>(a);
}

extern "C" __global__ __launch_bounds__(256) void attention_part_f32_512(AttnArgs a)
{
  attention_part_t<false, 4>(a);
}

// y = sum_s exp(m_s - M) acc_s / (sum_s exp(m_s - M) l_s + exp(sink - M)),
// M the largest range maximum (and the sink), over the splits ranges of one
// (head, row) at b (each hd values, its maximum, its sum); y the head's hd
// outputs. Every thread of the block calls it (at least 64 threads, splits
// <= 256).
template <bool AG = false>
__device__ __forceinline__ void merge_ranges(const double* b, int splits, int d, const float* sink,
                                             float* y, bool xcd = false)
{
  // AG: the ranges were written by other blocks of this launch (xcd: blocks
  // of this XCD, through its L2; else agent-scope)
  auto rd = [&](int i) { return AG ? (xcd ? load_xcd(b + i) : load_agent(b + i)) : b[i]; };
  // the range weights exp(m_s - M) and the range sums in LDS; the sums in
  // range order. Every load of the first MU ranges (a thread's dimension of
  // each, the maxima and sums) is issued before the first arithmetic: one
  // memory round trip.
  constexpr int MU = 16;
  __shared__ double wts[256], lsum[256];
  __shared__ double dsh[2];
  const int t = threadIdx.x;
  const int ic = min(t, d - 1);
  double pv[MU];
#pragma unroll
  for (int u = 0; u < MU; u++) pv[u] = rd(min(u, splits - 1) * (d + 2) + ic);
  // wave 0: the maxima, the weights and the denominator (a wave sum of the
  // weighted range sums), one barrier before the weighted values
  if (t < 64) {
    double M = -1.0e308;
    for (int s = t; s < splits; s += 64) {
      const double ms = rd(s * (d + 2) + d);
      wts[s] = ms;
      lsum[s] = rd(s * (d + 2) + d + 1);
      M = fmax(M, ms);
    }
    M = wave_max(M);
    if (sink && (double)*sink > M) M = *sink;
    double den = 0;
    for (int s = t; s < splits; s += 64) {
      const double ms = wts[s];
      const double e = ms > -1.0e308 ? exp(ms - M) : 0.0;
      wts[s] = e;
      den = __builtin_fma(e, lsum[s], den);
    }
    den = wave_sum(den, 64);
    if (sink) den = den + exp((double)*sink - M);
    if (t == 0) dsh[1] = 1.0 / den;
  }
  __syncthreads();
  const double inv = dsh[1];
  for (int i = t; i < d; i += blockDim.x) {
    double acc = 0;
    if (i == t) {
#pragma unroll
      for (int u = 0; u < MU; u++)
        if (u < splits) acc = acc + wts[u] * pv[u];
      for (int s = MU; s < splits; s++) acc = acc + wts[s] * rd(s * (d + 2) + i);
    } else {
      for (int s = 0; s < splits; s++) acc = acc + wts[s] * rd(s * (d + 2) + i);
    }
    y[i] = (float)(acc * inv);
  }
}

// one block per (head, row)
extern "C" __global__ __launch_bounds__(256) void attention_merge(AttnArgs a)
{
  const int h = blockIdx.x, r = blockIdx.y;
  const int d = a.hd;
  merge_ranges(a.part + ((int64_t)h * a.rows + r) * a.splits * (d + 2), a.splits, d,
               a.sinks ? a.sinks + h : nullptr, a.y + (int64_t)r * a.heads * d + (int64_t)h * d);
}

// ------------------------------------------------------------------- MoE
// ------------------------------------------------- attention of one row
// The decode step's attention ranges in one launch per layer: per (head,
// range of ATT_CHUNK keys) block, the Q/K head RMSNorm and RoPE of qkrope (the
// new key and value also stored into the cache by the blocks that hold
// them) and the range's partial softmax of attention_part; attention_merge
// adds the ranges. Every global load of a block - q, the new k/v, its keys
// and its values - is issued before the first arithmetic.
struct AttnOneArgs {
  const float* q;   // the row's q [heads * hd], k and v [kvh * hd] (GEMV outputs)
  const float* k;
  const float* v;
  const float* qn;  // head norms [hd] or null
  const float* kn;
  const float* cs;  // cos [hd / 2] then sin [hd / 2], or null: a NoPE layer
  void* kc;
  void* vc;
  float* y;         // [heads * hd]
  const float* sinks;
  const int* pastp;  // device position of the row (graph replay), or null: past
  double* part;      // [heads, splits, hd + 2]
  double scale, eps;
  int32_t heads, kvh, hd, past, window, splits;
  // [heads] counters 128 bytes apart (h * 32: one L2 line each), zero between
  // launches, or null: with them the last
  // range block of a head to finish merges the head's ranges (and sets its
  // counter back to zero), else attention_merge does
  int* done;  int32_t place, pad;  // f16 one-row launch: 0 blocks by head, 1 by KV group over the XCDs
};

// a head whose keys all fall in one range (cnt <= the range size): its range
// block writes the output itself, no partials, no counter, no merge; the
// arithmetic is merge_ranges' for one non-empty range (its weight exp(m - M)
// with the sink in M, the denominator fma(e, l, 0) plus the sink's term, each
// value 0 + e p, times 1 / den), so the bits are those of the merged path.
// m: the range's maximum score, l: its sum of weights, p(i): its weighted
// value sum of dimension i.
template <typename P>
__device__ __forceinline__ void finish_one_range(double m, double l, P p, int d, const float* sink,
                                                 float* y)
{
  double M = m;
  if (sink && (double)*sink > M) M = *sink;
  const double e = m > -1.0e308 ? exp(m - M) : 0.0;
  double den = __builtin_fma(e, l, 0.0);
  if (sink) den = den + exp((double)*sink - M);
  const double inv = 1.0 / den;
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    const double acc = 0.0 + e * p(i);
    y[i] = (float)(acc * inv);
  }
}

// the sums of two values over a block of 256 (wave sums, then 4 waves)
__device__ __forceinline__ void block_sum2(double& a, double& b, double* red)
{
  a = wave_sum(a, 64);
  b = wave_sum(b, 64);
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = a;
    red[4 + (threadIdx.x >> 6)] = b;
  }
  __syncthreads();
  a = (red[0] + red[1]) + (red[2] + red[3]);
  b = (red[4] + red[5]) + (red[6] + red[7]);
  __syncthreads();
}

template <bool F16, int HD>
__device__ __forceinline__ void attention_one_t(const AttnOneArgs& a)
{
  IHIP_STAMP_SCOPE;
  __shared__ double qd[HD];
  __shared__ float nq[HD], nk[HD];
  __shared__ float knew[HD], vnew[HD];
  __shared__ double sc[ATT_CHUNK];
  __shared__ double red[8];
  __shared__ double accs[4][HD];
  const int h = xcd_head(blockIdx.x, a.heads);
  const int s = blockIdx.z, t = threadIdx.x;
  constexpr int d = HD, half = HD / 2;
  IHIP_STAMP(0);
  const int64_t kvw = (int64_t)a.kvh * d;
  const int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  const int total = past + 1;
  const int first = (a.window > 0 && total > a.window) ? total - a.window : 0;
  const int cnt = total - first;
  const int j0 = min(cnt, s * ATT_CHUNK), j1 = min(cnt, j0 + ATT_CHUNK);
  const int n = j1 - j0;
  const int jn = cnt - 1 - j0;  // the new key within the range (valid when hasnew)
  const bool hasnew = n > 0 && j1 == cnt;
  // every key in range 0 (a short context, a window): that block finishes the
  // head alone (finish_one_range), the other ranges have nothing to add
  const bool whole = a.done && cnt <= ATT_CHUNK;
  if (whole && s > 0) return;
  double* out = a.part + ((int64_t)h * a.splits + s) * (d + 2);
  const int64_t base = (int64_t)(first + j0) * kvw + (int64_t)g * d;
  const int w = t >> 6, l = t & 63;
  constexpr int lpk = HD / 2;      // value pass: lanes per key (a dimension pair each)
  constexpr int kpw = 64 / lpk;     // keys side by side in a wave
  const int lane_key = l / lpk, pair = l % lpk;
  constexpr int step = 4 * kpw;
  constexpr int VB = ATT_CHUNK / step;            // a lane's keys: the whole range at once
  constexpr int KB = HD * (F16 ? 2 : 4) / 16;     // 16-byte loads of a key row

  // ---- every load first, each from a valid address (a clamped index; the
  // value of a key or lane past the end is not used), so that no load waits
  // for another
  const int tc = min(t, d - 1), th = min(t, half - 1);
  float qv = a.q[(int64_t)h * d + tc];
  const float qw = a.qn ? a.qn[tc] : 1.f;
  float kv = a.k[(int64_t)g * d + tc];
  const float vv = a.v[(int64_t)g * d + tc];
  const float kw = a.kn ? a.kn[tc] : 1.f;
  const bool rope = a.cs != nullptr;  // (null: a NoPE layer, q and k as normed)
  const float cv = rope ? a.cs[th] : 1.f, sv = rope ? a.cs[half + th] : 0.f;
  if (t >= d) qv = kv = 0.f;
  // the range's rows (an empty range reads row 0 of the cache)
  const int64_t rbase = n > 0 ? base : (int64_t)g * d;
  const int nmax = max(n - 1, 0);
  // f16 keys: the range's rows loaded coalesced (KROW lanes a row), turned
  // around in LDS (rows padded to an odd number of 16-byte words, so the
  // per-thread row reads hit distinct banks); f32 keys: a thread loads its row
  constexpr int KROW = HD * 2 / 16;              // 16-byte words of an f16 key row
  constexpr int KLD = ATT_CHUNK * KROW / 256;    // coalesced loads per thread
  constexpr int KPAD = KROW + 1;
  __shared__ uint4 ks[F16 ? ATT_CHUNK * KPAD : 1];
  uint4 kr[F16 ? KLD : KB];
  if constexpr (F16) {
#pragma unroll
    for (int r = 0; r < KLD; r++) {
      const int q = t + 256 * r, row = q / KROW, col = q % KROW;
      kr[r] = *(const uint4*)((const uint16_t*)a.kc + rbase + (int64_t)min(row, nmax) * kvw + col * 8);
    }

  } else {
    const uint4* p = (const uint4*)((const float*)a.kc + rbase + (int64_t)min(t, nmax) * kvw);
#pragma unroll
    for (int k = 0; k < KB; k++) kr[k] = p[k];
  }
  uint32_t vr[VB][F16 ? 1 : 2];
  const int jb0 = w * kpw + lane_key;
#pragma unroll
  for (int u = 0; u < VB; u++) {
    const int64_t e = rbase + (int64_t)min(jb0 + u * step, nmax) * kvw + 2 * pair;
    if constexpr (F16) {
      vr[u][0] = *(const uint32_t*)((const uint16_t*)a.vc + e);
    } else {
      uint2 x = *(const uint2*)((const float*)a.vc + e);
      vr[u][0] = x.x;
      vr[u][1] = x.y;
    }
  }
  // the key words into LDS once they arrive (the value loads are already out)
  if constexpr (F16) {
#pragma unroll
    for (int r = 0; r < KLD; r++) {
      const int q = t + 256 * r;
      ks[(q / KROW) * KPAD + q % KROW] = kr[r];
    }
  }

  IHIP_STAMP(1);
  // ---- the head norms (qkrope's arithmetic) and RoPE of q and the new key
  {
    double sq = (double)qv * (double)qv, sk = (double)kv * (double)kv;
    if (t >= d) sq = sk = 0;
    if (a.qn || (hasnew && a.kn)) block_sum2(sq, sk, red);
    float xq = qv, xk = kv;
    if (a.qn) xq = qw * (float)((double)qv * (1.0 / sqrt(sq / (double)d + a.eps)));
    if (hasnew && a.kn) xk = kw * (float)((double)kv * (1.0 / sqrt(sk / (double)d + a.eps)));
    if (t < d) {
      nq[t] = xq;
      nk[t] = xk;
    }
    __syncthreads();
    if (t < half) {
      double x0 = nq[t], x1 = nq[t + half], c = cv, sn = sv;
      qd[t] = rope ? (double)(float)(x0 * c - x1 * sn) : x0;
      qd[t + half] = rope ? (double)(float)(x1 * c + x0 * sn) : x1;
      if (hasnew) {
        double k0 = nk[t], k1 = nk[t + half];
        float o0 = rope ? (float)(k0 * c - k1 * sn) : (float)k0;
        float o1 = rope ? (float)(k1 * c + k0 * sn) : (float)k1;
        const int64_t dst = (int64_t)past * kvw + (int64_t)g * d;
        if constexpr (F16) {
          uint16_t h0 = float_to_half(o0), h1 = float_to_half(o1);
          ((uint16_t*)a.kc)[dst + t] = h0;
          ((uint16_t*)a.kc)[dst + t + half] = h1;
          // and into the range's key tile, as the cache now holds it
          uint16_t* kt = (uint16_t*)&ks[jn * KPAD];
          kt[t] = h0;
          kt[t + half] = h1;
          o0 = half_to_float(h0);
          o1 = half_to_float(h1);
        } else {
          ((float*)a.kc)[dst + t] = o0;
          ((float*)a.kc)[dst + t + half] = o1;
        }
        knew[t] = o0;
        knew[t + half] = o1;
      }
    }
    if (hasnew && t < d) {
      const int64_t dst = (int64_t)past * kvw + (int64_t)g * d;
      float x = vv;
      if constexpr (F16) {
        uint16_t hv = float_to_half(x);
        ((uint16_t*)a.vc)[dst + t] = hv;
        x = half_to_float(hv);
      } else {
        ((float*)a.vc)[dst + t] = x;
      }
      vnew[t] = x;
    }
    __syncthreads();
  }

  // ---- scores: the double dot per key. q and k are float values, so each
  // product is exact in double and a fused multiply-add rounds as the CPU's
  // multiply-then-add; the sum runs in interleaved chains (only the order of
  // the double sum differs from the CPU's). f16 keys: two threads per key,
  // each half of the dimensions, from the LDS key tile (the new key in it);
  // f32 keys: a thread per key from its registers.
  IHIP_STAMP(2);
  double m = -1.0e308;
  if constexpr (F16) {
    const int kk = t >> 1, hh = t & 1;
    double c4[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KROW / 2; k++) {
      const int kw = hh * (KROW / 2) + k;
      const uint4 kw4 = ks[kk * KPAD + kw];
      const uint32_t wv[4] = {kw4.x, kw4.y, kw4.z, kw4.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = 8 * kw + 2 * j;
        c4[(2 * j) & 3] = __builtin_fma(qd[i], (double)half_to_float(wv[j] & 0xffffu), c4[(2 * j) & 3]);
        c4[(2 * j + 1) & 3] =
            __builtin_fma(qd[i + 1], (double)half_to_float(wv[j] >> 16), c4[(2 * j + 1) & 3]);
      }
    }
    double part = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    double acc = part + xpart<1>(part);  // the other half of the key
    acc = acc * a.scale;
    if (kk < n) {
      if (hh == 0) sc[kk] = acc;
      m = acc;
    }
  } else if (t < n) {
    double c4[4] = {0, 0, 0, 0};
    if (hasnew && t == jn) {
#pragma unroll
      for (int i = 0; i < d; i++) c4[i & 3] = __builtin_fma(qd[i], (double)knew[i], c4[i & 3]);
    } else {
#pragma unroll
      for (int k = 0; k < KB; k++) {
        const uint32_t wv[4] = {kr[k].x, kr[k].y, kr[k].z, kr[k].w};
#pragma unroll
        for (int j = 0; j < 4; j++) c4[j] = __builtin_fma(qd[4 * k + j], (double)bits_float(wv[j]), c4[j]);
      }
    }
    double acc = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    acc = acc * a.scale;
    sc[t] = acc;
    m = acc;
  }
  __syncthreads();  // sc complete before the softmax reads it
  m = wave_max(m);
  if (l == 0) red[w] = m;
  __syncthreads();
  m = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
  double e = 0;
  if (t < n) {
    e = exp(sc[t] - m);
    sc[t] = e;
  } else if (t < ATT_CHUNK) {
    sc[t] = 0.0;  // no weight past the range: the value loop reads every slot
  }
  e = wave_sum(e, 64);
  __syncthreads();
  if (l == 0) red[4 + w] = e;

  IHIP_STAMP(3);
  // ---- the weighted values: the loads above, the new value from LDS
  // two chains per dimension (even and odd key slots); no branch: a slot
  // past the range has weight 0, the new key's value is selected
  const float vn0 = vnew[2 * pair], vn1 = vnew[2 * pair + 1];
  const int jnew = hasnew ? jn : -1;
  double a0e = 0, a1e = 0, a0o = 0, a1o = 0;
#pragma unroll
  for (int u = 0; u < VB; u++) {
    const int j = jb0 + u * step;
    const double p = sc[j];
    float x0, x1;
    if constexpr (F16) {
      x0 = half_to_float(vr[u][0] & 0xffffu);
      x1 = half_to_float(vr[u][0] >> 16);
    } else {
      x0 = bits_float(vr[u][0]);
      x1 = bits_float(vr[u][F16 ? 0 : 1]);
    }
    // a slot past the range reads a clamped row, which may be the new key's
    // not yet written one: its value is 0, never the row's bits
    x0 = j == jnew ? vn0 : (j < n ? x0 : 0.f);
    x1 = j == jnew ? vn1 : (j < n ? x1 : 0.f);
    if (u & 1) {
      a0o = __builtin_fma(p, (double)x0, a0o);
      a1o = __builtin_fma(p, (double)x1, a1o);
    } else {
      a0e = __builtin_fma(p, (double)x0, a0e);
      a1e = __builtin_fma(p, (double)x1, a1e);
    }
  }
  double a0 = a0e + a0o, a1 = a1e + a1o;
  if constexpr (lpk == 32) {  // the two keys of a wave: lanes l and l ^ 32
    a0 = a0 + xpart<32>(a0);
    a1 = a1 + xpart<32>(a1);
  }
  if (lane_key == 0) {
    accs[w][2 * pair] = a0;
    accs[w][2 * pair + 1] = a1;
  }
  __syncthreads();
  IHIP_STAMP(4);
  if (whole) {
    finish_one_range(n > 0 ? m : -1.0e308, (red[4] + red[5]) + (red[6] + red[7]),
                     [&](int i) { return (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]); }, d,
                     a.sinks ? a.sinks + h : nullptr, a.y + (int64_t)h * d);
    return;
  }
  // the head's last range block may read these: with a multiple of 8 heads
  // every range block of head h runs on one XCD (launch-order ids h' + heads
  // * s, xcd_head), so plain stores meet in that XCD's L2; else agent-scope
  const bool xcd = (a.heads & 7) == 0;
  auto put = [&](double* p, double v) {
    if (xcd) *p = v;
    else store_agent(p, v);
  };
  if (n > 0) {
    for (int i = t; i < d; i += 256) put(out + i, (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]));
    if (t == 0) {
      put(out + d, m);
      put(out + d + 1, (red[4] + red[5]) + (red[6] + red[7]));
    }
  } else if (t == 0) {  // an empty range: weight 0 in the merge
    put(out + d, -1.0e308);
    put(out + d + 1, 0.0);
  }
  // the head's last range block to finish merges the head's ranges
  if (a.done && last_block(a.done + h * 32, a.splits, xcd)) {
    IHIP_STAMP(5);
    merge_ranges<true>(a.part + (int64_t)h * a.splits * (d + 2), a.splits, d,
                       a.sinks ? a.sinks + h : nullptr, a.y + (int64_t)h * d, xcd);
    IHIP_STAMP(6);
    if (t == 0) a.done[h * 32] = 0;
  }
}

// ---------------------------------------------- the f16 decode attention
// The f16-cache decode step of attention_one_t, its arithmetic bit for bit,
// with the launch laid out for the chip:
//  - blocks by KV group: the 1-D grid's block lin runs on XCD lin % 8, and
//    XCD c takes KV group c / X (X = 8 / kvh XCDs a group) over every X-th
//    key range, all heads of the group: each key and value tile is fetched
//    into one L2 (by head, a group's heads spanned two XCDs and both L2s
//    fetched its tiles);
//  - the range's keys and values through buffer loads bounded by the range's
//    rows (a row past them, and the new key's row not yet written, reads 0):
//    no per-load 64-bit address or clamp, no per-key select;
//  - the head norms and RoPE in wave 0 alone (a lane holds the pairs of its
//    dimensions: no block reduction), while the tiles are on their way.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bounded(const void* p, uint32_t bytes)
{
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// block lin of heads * splits: its head, its range, and whether every range
// block of the head runs on one XCD (its partials then meet in that L2)
__device__ __forceinline__ void attn_one_block(int lin, int heads, int kvh, int splits, int& h,
                                               int& s, bool& xcd, int place)
{
  if (place == 0 && (heads & 7) == 0) {
    // by head: XCD c takes heads c * heads / 8 .. over every range
    h = xcd_head((unsigned)(lin % heads), heads);
    s = lin / heads;
    xcd = true;
  } else if ((heads & 7) == 0 && kvh <= 8 && (8 % kvh) == 0) {
    const int X = 8 / kvh, hpg = heads / kvh;  // the host rounds splits to a multiple of X
    const int c = lin & 7, r = lin >> 3;
    h = (c / X) * hpg + r % hpg;
    s = (r / hpg) * X + c % X;
    xcd = X == 1;
  } else {
    h = lin % heads;
    s = lin / heads;
    xcd = false;
  }
  (void)splits;
}

template <int HD>
__device__ __forceinline__ void attention_one_f16(const AttnOneArgs& a)
{
  IHIP_STAMP_SCOPE;
  constexpr int d = HD, half = HD / 2;
  constexpr int QPL = HD / 64;                  // dimensions of the head per lane of wave 0
  constexpr int KROW = HD * 2 / 16;             // 16-byte words of a key row
  constexpr int KLD = ATT_CHUNK * KROW / 256;   // key words per thread
  constexpr int KPAD = KROW + 1;                // odd row pitch: the per-key reads hit distinct banks
  constexpr int lpk = HD / 2;                   // value pass: lanes per key (a dimension pair each)
  constexpr int kpw = 64 / lpk;                 // keys side by side in a wave
  constexpr int step = 4 * kpw;
  constexpr int VB = ATT_CHUNK / step;          // a lane's keys
  __shared__ double qd[HD];
  __shared__ double sc[ATT_CHUNK];
  __shared__ double red[8];
  __shared__ double accs[4][HD];
  __shared__ uint4 ks[ATT_CHUNK * KPAD];
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  int h, s;
  bool xcd;
  attn_one_block(blockIdx.x, a.heads, a.kvh, a.splits, h, s, xcd, a.place);
  IHIP_STAMP(0);
  const int kvw = a.kvh * d;
  const uint32_t rowb = (uint32_t)kvw * 2u;  // bytes of a cache row
  const int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  const int total = past + 1;
  const int first = (a.window > 0 && total > a.window) ? total - a.window : 0;
  const int cnt = total - first;
  const int j0 = min(cnt, s * ATT_CHUNK), j1 = min(cnt, j0 + ATT_CHUNK);
  const int n = j1 - j0;
  const bool hasnew = n > 0 && j1 == cnt;  // the range holds the new key, its last row
  const int jn = n - 1;
  const int nload = hasnew ? n - 1 : n;    // rows already in the cache
  // every key in range 0 (a short context, a window): that block finishes the
  // head alone (finish_one_range), the other ranges have nothing to add
  const bool whole = a.done && cnt <= ATT_CHUNK;
  if (whole && s > 0) return;
  double* out = a.part + ((int64_t)h * a.splits + s) * (d + 2);
  const int64_t rbase = (int64_t)(first + j0) * kvw + (int64_t)g * d;  // halves
  const auto kr = bounded((const uint16_t*)a.kc + rbase, (uint32_t)nload * rowb);
  const auto vr = bounded((const uint16_t*)a.vc + rbase, (uint32_t)nload * rowb);
  const int lane_key = l / lpk, pair = l % lpk;
  const int jb0 = w * kpw + lane_key;  // value pass: key jb0 + u * step

  // ---- every load first: wave 0 the head's q (and the new key), every
  // thread its key words and value pairs
  float qv[QPL], qw[QPL], kv[QPL], kw[QPL], cv[QPL], sv[QPL];
  if (w == 0) {
#pragma unroll
    for (int i = 0; i < QPL; i++) {
      const int e = l + 64 * i, p = e % half;
      qv[i] = a.q[(int64_t)h * d + e];
      qw[i] = a.qn ? a.qn[e] : 1.f;
      kv[i] = hasnew ? a.k[(int64_t)g * d + e] : 0.f;
      kw[i] = (hasnew && a.kn) ? a.kn[e] : 1.f;
      cv[i] = a.cs ? a.cs[p] : 1.f;  // (null: a NoPE layer)
      sv[i] = a.cs ? a.cs[half + p] : 0.f;
    }
  }
  uint4 kt[KLD];
  const uint32_t koff = (uint32_t)(t / KROW) * rowb + (uint32_t)(t % KROW) * 16u;
#pragma unroll
  for (int r = 0; r < KLD; r++)
    kt[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                          kr, (int)(koff + (uint32_t)r * (256u / KROW) * rowb), 0, 0));
  uint32_t vv[VB];
  const uint32_t voff = (uint32_t)jb0 * rowb + (uint32_t)pair * 4u;
#pragma unroll
  for (int u = 0; u < VB; u++)
    vv[u] = __builtin_amdgcn_raw_buffer_load_b32(vr, (int)(voff + (uint32_t)(u * step) * rowb), 0, 0);
  // the new value (its f16 bits, as the cache holds it) for the wave and
  // lanes whose chain holds the new key
  const bool vlane = hasnew && w == (jn % step) / kpw && lane_key == (jn % kpw);
  float vn0 = 0.f, vn1 = 0.f;
  if (vlane) {
    const float2 x = *(const float2*)(a.v + (int64_t)g * d + 2 * pair);
    const uint16_t h0 = float_to_half(x.x), h1 = float_to_half(x.y);
    vn0 = half_to_float(h0);
    vn1 = half_to_float(h1);
    ((uint32_t*)a.vc)[((int64_t)past * kvw + (int64_t)g * d) / 2 + pair] = (uint32_t)h0 | ((uint32_t)h1 << 16);
  }
  IHIP_STAMP(1);

  // ---- wave 0: the head norms (qkrope's arithmetic: the sums of squares
  // of dimensions 0..63 and 64..127 as the two waves of a block formed
  // them) and RoPE of q and the new key
  if (w == 0) {
    double sqa = (double)qv[0] * (double)qv[0], ska = (double)kv[0] * (double)kv[0];
    double sq = wave_sum(sqa, 64), sk = wave_sum(ska, 64);
    if constexpr (QPL == 2) {
      const double sqb = (double)qv[1] * (double)qv[1], skb = (double)kv[1] * (double)kv[1];
      sq = sq + wave_sum(sqb, 64);
      sk = sk + wave_sum(skb, 64);
    }
    float xq[QPL], xk[QPL];
#pragma unroll
    for (int i = 0; i < QPL; i++) {
      xq[i] = qv[i];
      xk[i] = kv[i];
      if (a.qn) xq[i] = qw[i] * (float)((double)qv[i] * (1.0 / sqrt(sq / (double)d + a.eps)));
      if (hasnew && a.kn) xk[i] = kw[i] * (float)((double)kv[i] * (1.0 / sqrt(sk / (double)d + a.eps)));
    }
    // the pair (p, p + half): in one lane (HD 128), in lanes l and l ^ 32 (HD 64)
    double x0, x1, k0, k1;
    if constexpr (QPL == 2) {
      x0 = xq[0]; x1 = xq[1]; k0 = xk[0]; k1 = xk[1];
    } else {
      const float pq = xpart<32>(xq[0]), pk = xpart<32>(xk[0]);
      const bool lo = l < half;
      x0 = lo ? xq[0] : pq; x1 = lo ? pq : xq[0];
      k0 = lo ? xk[0] : pk; k1 = lo ? pk : xk[0];
    }
    const double c = cv[0], sn = sv[0];
    const bool rope = a.cs != nullptr;  // (a NoPE layer: q and the new key as normed)
    const double r0 = rope ? (double)(float)(x0 * c - x1 * sn) : x0;
    const double r1 = rope ? (double)(float)(x1 * c + x0 * sn) : x1;
    const float o0 = rope ? (float)(k0 * c - k1 * sn) : (float)k0;
    const float o1 = rope ? (float)(k1 * c + k0 * sn) : (float)k1;
    uint16_t* knew = (uint16_t*)&ks[jn * KPAD];
    const int64_t dst = (int64_t)past * kvw + (int64_t)g * d;
    if constexpr (QPL == 2) {
      qd[l] = r0;
      qd[l + 64] = r1;
      if (hasnew) {
        const uint16_t h0 = float_to_half(o0), h1 = float_to_half(o1);
        ((uint16_t*)a.kc)[dst + l] = h0;
        ((uint16_t*)a.kc)[dst + l + 64] = h1;
        knew[l] = h0;
        knew[l + 64] = h1;
      }
    } else {
      const bool lo = l < half;
      qd[l] = lo ? r0 : r1;
      if (hasnew) {
        const uint16_t hk = float_to_half(lo ? o0 : o1);
        ((uint16_t*)a.kc)[dst + l] = hk;
        knew[l] = hk;
      }
    }
  }
  // the key words into LDS (the new key's row is wave 0's)
#pragma unroll
  for (int r = 0; r < KLD; r++) {
    const int q = t + 256 * r, row = q / KROW;
    if (!(hasnew && row == jn)) ks[row * KPAD + q % KROW] = kt[r];
  }
  __syncthreads();

  // ---- scores (attention_one_t's): two threads a key, four chains each
  IHIP_STAMP(2);
  double m = -1.0e308;
  {
    const int kk = t >> 1, hh = t & 1;
    double c4[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KROW / 2; k++) {
      const int kw2 = hh * (KROW / 2) + k;
      const uint4 kw4 = ks[kk * KPAD + kw2];
      const uint32_t wv[4] = {kw4.x, kw4.y, kw4.z, kw4.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = 8 * kw2 + 2 * j;
        c4[(2 * j) & 3] = __builtin_fma(qd[i], (double)half_to_float(wv[j] & 0xffffu), c4[(2 * j) & 3]);
        c4[(2 * j + 1) & 3] =
            __builtin_fma(qd[i + 1], (double)half_to_float(wv[j] >> 16), c4[(2 * j + 1) & 3]);
      }
    }
    const double part = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    double acc = part + xpart<1>(part);
    acc = acc * a.scale;
    if (kk < n) {
      if (hh == 0) sc[kk] = acc;
      m = acc;
    }
  }
  __syncthreads();
  m = wave_max(m);
  if (l == 0) red[w] = m;
  __syncthreads();
  m = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
  double e = 0;
  if (t < n) {
    e = exp(sc[t] - m);
    sc[t] = e;
  } else if (t < ATT_CHUNK) {
    sc[t] = 0.0;
  }
  e = wave_sum(e, 64);
  __syncthreads();
  if (l == 0) red[4 + w] = e;

  // ---- the weighted values: even and odd key slots in two chains per
  // dimension; a row past the range read 0 (weight 0), the new key's value
  // added after its chain's last nonzero term, where its slot puts it
  IHIP_STAMP(3);
  double a0e = 0, a1e = 0, a0o = 0, a1o = 0;
#pragma unroll
  for (int u = 0; u < VB; u++) {
    const double p = sc[jb0 + u * step];
    const double x0 = half_to_float(vv[u] & 0xffffu), x1 = half_to_float(vv[u] >> 16);
    if (u & 1) {
      a0o = __builtin_fma(p, x0, a0o);
      a1o = __builtin_fma(p, x1, a1o);
    } else {
      a0e = __builtin_fma(p, x0, a0e);
      a1e = __builtin_fma(p, x1, a1e);
    }
  }
  if (vlane) {
    const double p = sc[jn];
    if ((jn / step) & 1) {
      a0o = __builtin_fma(p, (double)vn0, a0o);
      a1o = __builtin_fma(p, (double)vn1, a1o);
    } else {
      a0e = __builtin_fma(p, (double)vn0, a0e);
      a1e = __builtin_fma(p, (double)vn1, a1e);
    }
  }
  double a0 = a0e + a0o, a1 = a1e + a1o;
  if constexpr (lpk == 32) {
    a0 = a0 + xpart<32>(a0);
    a1 = a1 + xpart<32>(a1);
  }
  if (lane_key == 0) {
    accs[w][2 * pair] = a0;
    accs[w][2 * pair + 1] = a1;
  }
  __syncthreads();
  IHIP_STAMP(4);
  if (whole) {
    finish_one_range(n > 0 ? m : -1.0e308, (red[4] + red[5]) + (red[6] + red[7]),
                     [&](int i) { return (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]); }, d,
                     a.sinks ? a.sinks + h : nullptr, a.y + (int64_t)h * d);
    return;
  }
  auto put = [&](double* p, double v) {
    if (xcd) *p = v;
    else store_agent(p, v);
  };
  if (n > 0) {
    for (int i = t; i < d; i += 256) put(out + i, (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]));
    if (t == 0) {
      put(out + d, m);
      put(out + d + 1, (red[4] + red[5]) + (red[6] + red[7]));
    }
  } else if (t == 0) {
    put(out + d, -1.0e308);
    put(out + d + 1, 0.0);
  }
  if (a.done && last_block(a.done + h * 32, a.splits, xcd)) {
    IHIP_STAMP(5);
    merge_ranges<true>(a.part + (int64_t)h * a.splits * (d + 2), a.splits, d,
                       a.sinks ? a.sinks + h : nullptr, a.y + (int64_t)h * d, xcd);
    IHIP_STAMP(6);
    if (t == 0) a.done[h * 32] = 0;
  }
}

extern "C" __global__ __launch_bounds__(256, 1) void attention_one_f16_64(AttnOneArgs a)
{
  ihip::touch_kernargs<sizeof(AttnOneArgs)>();
  attention_one_f16<64>(a);
}
extern "C" __global__ __launch_bounds__(256, 1) void attention_one_f16_128(AttnOneArgs a)
{
  ihip::touch_kernargs<sizeof(AttnOneArgs)>();
  attention_one_f16<128>(a);
}
extern "C" __global__ __launch_bounds__(256, 1) void attention_one_f32_64(AttnOneArgs a)
{
  ihip::touch_kernargs<sizeof(AttnOneArgs)>();
  attention_one_t<false, 64>(a);
}
extern "C" __global__ __launch_bounds__(256, 1) void attention_one_f32_128(AttnOneArgs a)
{
  ihip::touch_kernargs<sizeof(AttnOneArgs)>();
  attention_one_t<false, 128>(a);
}

// the split sums of the float-weight GEMM (gemm_flt with ksplit > 1): y[r,
// o] = bias[o] + the ksplit double partial sums of (r, o) in split order,
// rounded to single
struct SplitSumArgs {
  const double* part;  // [ksplit, rows, out]
  const float* bias;   // [out] or null
  float* y;            // [rows, out]
  int64_t n;           // rows * out
  int32_t out, ksplit;
};

extern "C" __global__ __launch_bounds__(256) void gemm_split_sum(SplitSumArgs a)
{
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  double v = a.part[i];
  for (int z = 1; z < a.ksplit; z++) v = v + a.part[(int64_t)z * a.n + i];
  if (a.bias) v = (double)a.bias[i % a.out] + v;
  a.y[i] = (float)v;
}

struct RouteArgs {
  const float* logits;
  int* ids;
  float* w;
  int32_t experts, k, norm, rows;
  const float* scale;  // [experts]: each weight times its expert's (Gemma 4), or null
};

// one block of 256 per row (route_block of route.h)
extern "C" __global__ __launch_bounds__(256) void route(RouteArgs a)
{
  __shared__ int sid[64];
  __shared__ float sw[64];
  const int row = blockIdx.x;
  route_block<4096>(a.logits + (int64_t)row * a.experts, a.experts, a.k, a.norm, sid, sw);
  if ((int)threadIdx.x < a.k) {
    float w = sw[threadIdx.x];
    if (a.scale) w = w * a.scale[sid[threadIdx.x]];
    a.ids[(int64_t)row * a.k + threadIdx.x] = sid[threadIdx.x];
    a.w[(int64_t)row * a.k + threadIdx.x] = w;
  }
}

struct CombineArgs {
  const float* d;  // [rows * k, n]
  const float* w;  // [rows * k]
  float* y;        // [rows, n]
  int32_t k, n, rows, pad;
};

// y = sum over the k slots, in slot (= id) order, of w[s] * d[s]: the
// single-rounded steps of TDecoderModel.Experts (decoder.pas:3140-3148)
extern "C" __global__ __launch_bounds__(256) void moecombine(CombineArgs a)
{
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int row = blockIdx.y;
  if (i >= a.n) return;
  float acc = 0.f;
  for (int s = 0; s < a.k; s++) {
    float p = a.w[(int64_t)row * a.k + s] * a.d[((int64_t)row * a.k + s) * a.n + i];
    acc = acc + p;
  }
  a.y[(int64_t)row * a.n + i] = acc;
}

// ------------------------------------------------------------------ argmax
struct ArgmaxArgs {
  const float* v;
  int* out;
  int64_t n;
  uint64_t* part;  // [parts] block results
  int64_t chunk;   // values per block of argmax_part
  int32_t parts, pad;
};

// InferArgMax (sampler.pas:123-160): the float bits ordered as integers (the
// lower 31 flipped when negative, -0 as +0), NaN skipped, the first index of
// the maximum; all NaN gives 0. A candidate is packed into one uint64 - the
// key (sign flipped) above the inverted index - so the largest packed value
// is the largest key at its lowest index, and 0 is "no candidate".
__device__ __forceinline__ uint64_t argmax_pack(float f, int64_t i)
{
  uint32_t b = float_bits(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0;  // NaN
  int k = (int)(b ^ ((b >> 31) * 0x7fffffffu));
  if (k == -1) k = 0;
  return ((uint64_t)((uint32_t)k ^ 0x80000000u) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* sh)
{
  uint64_t o;
  o = xpart<1>(v); v = o > v ? o : v;
  o = xpart<2>(v); v = o > v ? o : v;
  o = xpart<4>(v); v = o > v ? o : v;
  o = xpart<8>(v); v = o > v ? o : v;
  o = xpart<16>(v); v = o > v ? o : v;
  o = xpart<32>(v); v = o > v ? o : v;
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  v = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) v = sh[i] > v ? sh[i] : v;
  return v;
}

// stage 1: block b reduces values [b chunk, (b + 1) chunk)
extern "C" __global__ __launch_bounds__(256) void argmax_part(ArgmaxArgs a)
{
  __shared__ uint64_t sh[4];
  const int64_t i0 = (int64_t)blockIdx.x * a.chunk;
  const int64_t i1 = min(a.n, i0 + a.chunk);
  uint64_t best = 0;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
    uint64_t c = argmax_pack(a.v[i], i);
    best = c > best ? c : best;
  }
  best = block_max_u64(best, sh);
  if (threadIdx.x == 0) a.part[blockIdx.x] = best;
}

// stage 2: the block results
extern "C" __global__ __launch_bounds__(256) void argmax_final(ArgmaxArgs a)
{
  __shared__ uint64_t sh[4];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < a.parts; i += 256) best = a.part[i] > best ? a.part[i] : best;
  best = block_max_u64(best, sh);
  if (threadIdx.x == 0) a.out[0] = best ? (int)(0xffffffffu - (uint32_t)best) : 0;
}

// ------------------------------------------------------------------ sampling
// TInferSampler.Next (sampler.pas:269-435) for one row of logits: the softmax
// of logits / temperature in double, then either one draw over every token in
// id order, or the warpers in the order of generate() - top-k keeping the ties
// of the k-th logit, top-p over what top-k kept, min-p - and one draw from
// what is left, all in the order (logit descending, id ascending).
//
// The reference lowers a probability threshold until its candidates hold
// what the filters keep, sorts them and cuts the sorted list. What it keeps
// depends only on the filters, so here the candidates are any superset, and
// nothing is sorted:
// - sample_probs (a block per 'per' tokens): p = exp((l - max) / T), the
//   block's sum of p, and a histogram of p over 128 buckets (the binary
//   exponent and the first mantissa bit: larger p, lower bucket) with each
//   bucket's count and 40-bit fixed-point mass;
// - sample_compact: the bucket level L that surely holds what the filters
//   keep (k tokens, top_p of the mass, or the min-p cut), the same in every
//   block; each block writes its candidates (bucket <= L) in id order at its
//   offset. Without filters, each block's sum of p / sum instead.
// - sample_pick (one block): top-k is the key of the k-th logit (a radix
//   select), min-p the smallest key whose p / sum reaches min_p times the
//   best's (p grows with the logit), the top-p cut and the draw radix
//   searches of the running probability in (key descending, id ascending)
//   order over 8-bit key digits, with 62-bit fixed-point sums (exact integer
//   sums: the result does not depend on the order of atomics).
constexpr int SNT = 1024;   // threads of sample_pick
constexpr int SBT = 256;    // threads of sample_probs / sample_compact
constexpr int SBK = 128;    // buckets of p
struct SampleArgs {
  const float* logits;
  const int* best;     // the argmax of the row (InferArgMax)
  int* out;            // the drawn id (may be best)
  uint64_t* state;     // the splitmix64 state, advanced once per draw
  double* p;           // [n] exp((logit - max) / temperature), 0 for NaN / Inf
  double* bsum;        // [nb] the blocks' sums of p
  double* bq;          // [nb] the blocks' sums of p / sum (the unfiltered draw)
  uint32_t* bcnt;      // [nb][SBK] counts per bucket
  uint64_t* bmass;     // [nb][SBK] fixed-point masses per bucket (2^40 = p of 1)
  int* cid;            // [n] the candidates: id, logit key, p
  uint32_t* ckey;
  double* cp;
  double temperature, top_p, min_p;
  int32_t n, top_k, nb, per;
};

// the logit as an order-preserving key (-0 as +0), as argmax_pack
__device__ __forceinline__ uint32_t logit_key(float f)
{
  const uint32_t b = float_bits(f);
  int k = (int)(b ^ ((b >> 31) * 0x7fffffffu));
  if (k == -1) k = 0;
  return (uint32_t)k ^ 0x80000000u;
}

__device__ __forceinline__ bool finite_bits(float f) { return (float_bits(f) & 0x7f800000u) != 0x7f800000u; }

// the bucket of p in (0, 1] (2 per binary exponent, larger p lower); 0 in the last
__device__ __forceinline__ int p_bucket(double p)
{
  const uint64_t b = __builtin_bit_cast(uint64_t, p);
  const int e = 1023 - (int)((b >> 52) & 2047);  // 0 for [1, 2)
  const int hi = (int)((b >> 51) & 1);
  return p > 0.0 ? min(SBK - 1, max(0, 2 * e + 1 - hi)) : SBK - 1;
}

// splitmix64 (the published generator of Vigna): 53 random bits in [0, 1)
__device__ __forceinline__ double splitmix_next(uint64_t* state)
{
  uint64_t st = *state + 0x9E3779B97F4A7C15ull;
  *state = st;
  uint64_t z = st;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// block-wide sums, minima and exclusive prefixes in a fixed order (NT threads)
template <int NT, typename T>
__device__ __forceinline__ T sblock_sum(T v, T* sh)
{
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int o = NT / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) sh[threadIdx.x] = sh[threadIdx.x] + sh[threadIdx.x + o];
    __syncthreads();
  }
  const T r = sh[0];
  __syncthreads();
  return r;
}

template <int NT, typename T>
__device__ __forceinline__ T sblock_min(T v, T* sh)
{
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int o = NT / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) sh[threadIdx.x] = min(sh[threadIdx.x], sh[threadIdx.x + o]);
    __syncthreads();
  }
  const T r = sh[0];
  __syncthreads();
  return r;
}

template <int NT, typename T>
__device__ __forceinline__ T sblock_exclusive(T v, T* sh)
{
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int o = 1; o < NT; o <<= 1) {
    const T a = (int)threadIdx.x >= o ? sh[threadIdx.x - o] : T(0);
    __syncthreads();
    sh[threadIdx.x] = sh[threadIdx.x] + a;
    __syncthreads();
  }
  const T r = sh[threadIdx.x] - v;
  __syncthreads();
  return r;
}

constexpr double FX_ONE = 4611686018427387904.0;  // 2^62: a probability of 1
constexpr double MX_ONE = 1099511627776.0;        // 2^40: a p of 1 (bucket masses)

// the normalised probability p / sum as a 62-bit fixed-point weight: one
// definition for every sum and search, so their totals agree to the bit
__device__ __forceinline__ uint64_t wfx(double p, double sum) { return (uint64_t)(p / sum * FX_ONE); }

// no finite best, or a temperature too close to 0 to divide by: greedy
__device__ __forceinline__ bool sample_greedy(const SampleArgs& a, int best)
{
  return !finite_bits(a.logits[best]) || !(a.temperature >= 1e-30);
}

__device__ __forceinline__ bool sample_filters(const SampleArgs& a)
{
  return a.top_k > 0 || a.top_p < 1.0 || a.min_p > 0.0;
}

extern "C" __global__ __launch_bounds__(256) void sample_probs(SampleArgs a)
{
  __shared__ double shd[SBT];
  __shared__ uint32_t hc[SBK];
  __shared__ unsigned long long hm[SBK];
  const int t = threadIdx.x, b = blockIdx.x;
  const int best = *a.best;
  if (sample_greedy(a, best)) return;
  const bool filters = sample_filters(a);
  if (t < SBK) {
    hc[t] = 0;
    hm[t] = 0;
  }
  __syncthreads();
  const double m = a.logits[best], inv = 1.0 / a.temperature;
  const int ept = a.per / SBT;  // a contiguous run per thread
  const int i0 = min(a.n, b * a.per + t * ept), i1 = min(a.n, i0 + ept);
  double s = 0;
  for (int i = i0; i < i1; i++) {
    const float l = a.logits[i];
    const bool fin = finite_bits(l);
    const double p = fin ? exp(((double)l - m) * inv) : 0.0;
    a.p[i] = p;
    s = s + p;
    if (filters && fin) {
      const int k = p_bucket(p);
      atomicAdd(&hc[k], 1u);
      atomicAdd(&hm[k], (unsigned long long)(p * MX_ONE));
    }
  }
  s = sblock_sum<SBT>(s, shd);
  if (t == 0) a.bsum[b] = s;
  if (filters && t < SBK) {
    a.bcnt[(int64_t)b * SBK + t] = hc[t];
    a.bmass[(int64_t)b * SBK + t] = hm[t];
  }
}

// the sum of p over the blocks (at most 256): a tree in a fixed order over
// the block sums, the same value in every kernel that takes it
template <int NT>
__device__ __forceinline__ double blocks_sum(const SampleArgs& a, double* sh)
{
  if ((int)threadIdx.x < 256) sh[threadIdx.x] = (int)threadIdx.x < a.nb ? a.bsum[threadIdx.x] : 0.0;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) sh[threadIdx.x] = sh[threadIdx.x] + sh[threadIdx.x + o];
    __syncthreads();
  }
  const double r = sh[0];
  __syncthreads();
  return r;
}

// the count and fixed-point mass of every bucket over the blocks: each
// thread reads whole rows of blocks (16-byte loads, all in flight) and adds
// them into LDS (integer sums: the order does not matter)
template <int NT>
__device__ __forceinline__ void bucket_totals(const SampleArgs& a, uint32_t* cnt, uint64_t* mass, uint64_t* shu)
{
  (void)shu;
  const int t = threadIdx.x;
  if (t < SBK) {
    cnt[t] = 0;
    mass[t] = 0;
  }
  __syncthreads();
  // (block, quarter of its row): 32 buckets per item
  for (int it = t; it < a.nb * 4; it += NT) {
    const int b = it >> 2, k0 = (it & 3) * 32;
    const uint4* pc = (const uint4*)(a.bcnt + (int64_t)b * SBK + k0);
    const uint4* pm = (const uint4*)(a.bmass + (int64_t)b * SBK + k0);
    uint4 c[8], m[16];
#pragma unroll
    for (int x = 0; x < 8; x++) c[x] = pc[x];
#pragma unroll
    for (int x = 0; x < 16; x++) m[x] = pm[x];
#pragma unroll
    for (int x = 0; x < 8; x++) {
      const uint32_t v[4] = {c[x].x, c[x].y, c[x].z, c[x].w};
#pragma unroll
      for (int y = 0; y < 4; y++)
        if (v[y]) atomicAdd(&cnt[k0 + 4 * x + y], v[y]);
    }
#pragma unroll
    for (int x = 0; x < 16; x++) {
      const uint64_t v0 = ((uint64_t)m[x].y << 32) | m[x].x, v1 = ((uint64_t)m[x].w << 32) | m[x].z;
      if (v0) atomicAdd((unsigned long long*)&mass[k0 + 2 * x], (unsigned long long)v0);
      if (v1) atomicAdd((unsigned long long*)&mass[k0 + 2 * x + 1], (unsigned long long)v1);
    }
  }
  __syncthreads();
}

// the candidate bucket level (thread 0's loops; the same in every kernel):
// top-k: the first bucket whose running count reaches k; top-p alone: whose
// running mass reaches top_p of the sum (a margin for the fixed point); min-p
// alone: the bucket of its cut; else every finite token
__device__ int sample_level(const SampleArgs& a, const uint32_t* cnt, const uint64_t* mass, double sum)
{
  if (a.top_k > 0) {
    uint64_t c = 0;
    for (int k = 0; k < SBK; k++)
      if ((c += cnt[k]) >= (uint64_t)a.top_k) return k;
    return SBK - 1;
  }
  if (a.top_p < 1.0) {
    uint64_t c = 0;
    // the truncation of each token's fixed-point mass: at most n units short
    const double want = a.top_p * sum * (1.0 + 1e-9) * MX_ONE + (double)a.n + 1.0;
    for (int k = 0; k < SBK; k++)
      if ((double)(c += mass[k]) >= want) return k;
    return SBK - 1;
  }
  return p_bucket(a.min_p * (1.0 - 1e-9));
}

extern "C" __global__ __launch_bounds__(256) void sample_compact(SampleArgs a)
{
  __shared__ uint32_t cnt[SBK];
  __shared__ uint64_t mass[SBK];
  __shared__ uint64_t shu[SBT];
  __shared__ double shd[SBT];
  __shared__ int level;
  __shared__ uint64_t at0;
  const int t = threadIdx.x, b = blockIdx.x;
  const int best = *a.best;
  if (sample_greedy(a, best)) return;
  const int ept = a.per / SBT;
  const int i0 = min(a.n, b * a.per + t * ept), i1 = min(a.n, i0 + ept);
  const double sum = blocks_sum<SBT>(a, shd);
  if (!sample_filters(a)) {
    double q = 0;
    for (int i = i0; i < i1; i++) q = q + a.p[i] / sum;
    q = sblock_sum<SBT>(q, shd);
    if (t == 0) a.bq[b] = q;
    return;
  }
  // the totals per bucket over the blocks, then the level
  bucket_totals<SBT>(a, cnt, mass, shu);
  if (t == 0) level = sample_level(a, cnt, mass, sum);
  __syncthreads();
  const int L = level;
  // this block's offset: the candidates of the blocks before it
  uint64_t before = 0;
  for (int k = t; k < b; k += SBT) {
#pragma unroll 8
    for (int j = 0; j <= L; j++) before += a.bcnt[(int64_t)k * SBK + j];
  }
  before = sblock_sum<SBT>(before, shu);
  if (t == 0) at0 = before;
  __syncthreads();
  uint64_t mine = 0;
  for (int i = i0; i < i1; i++)
    if (finite_bits(a.logits[i]) && p_bucket(a.p[i]) <= L) mine++;
  uint64_t at = at0 + sblock_exclusive<SBT>(mine, shu);
  for (int i = i0; i < i1; i++) {
    const float l = a.logits[i];
    if (finite_bits(l) && p_bucket(a.p[i]) <= L) {
      a.cid[at] = i;
      a.ckey[at] = logit_key(l);
      a.cp[at] = a.p[i];
      at++;
    }
  }
}

// what the warpers kept: a key at or above kmin (top-k, min-p) and, after a
// top-p cut at (kp, ip), a key above kp or kp with an id up to ip
struct Kept {
  uint32_t kmin = 0;
  bool cut = false;
  uint32_t kp = 0;
  int ip = 0;
  __device__ bool operator()(uint32_t key, int id) const
  {
    return key >= kmin && !(cut && (key < kp || (key == kp && id > ip)));
  }
};

// the first candidate, in (key descending, id ascending) order among the kept
// ones, at which the running sum of the weights (the count 1 when ONE, else
// the fixed-point probability) reaches rem (>= rem, or > rem when strict).
// Returns the id, or -1 when the total stays short of rem. Per-wave
// histograms of the 256 digit values, added in wave order.
template <bool ONE>
__device__ int radix_search(const SampleArgs& a, const Kept& k, int nc, uint64_t rem, bool strict, double sum,
                            uint64_t (*hist)[256], uint64_t* shu, int* shi, uint32_t* found_key)
{
  __shared__ int choice;
  __shared__ uint64_t rem_sh;
  const int t = threadIdx.x, w = t >> 6;
  uint32_t prefix = 0, mask = 0;
  for (int d = 0; d < 4; d++) {
    const int shift = 24 - 8 * d;
    for (int x = t; x < 16 * 256; x += SNT) hist[x >> 8][x & 255] = 0;
    __syncthreads();
    for (int c = t; c < nc; c += SNT) {
      const uint32_t key = a.ckey[c];
      if ((key & mask) != prefix || !k(key, a.cid[c])) continue;
      const uint64_t wt = ONE ? 1ull : wfx(a.cp[c], sum);
      atomicAdd((unsigned long long*)&hist[w][(key >> shift) & 255u], (unsigned long long)wt);
    }
    __syncthreads();
    // the bins over the waves, then their sums from the top digit down
    // (S[d] = sum of bins >= d): the digit is the largest d whose S[d]
    // reaches rem, the rest carries S[d + 1]
    uint64_t h = 0;
    if (t < 256)
      for (int x = 0; x < 16; x++) h += hist[x][t];
    if (t == 0) choice = -1;
    __syncthreads();
    if (t < 256) hist[0][255 - t] = h;  // reversed: a prefix sum gives S
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const uint64_t v = (t < 256 && t >= o) ? hist[0][t - o] : 0ull;
      __syncthreads();
      if (t < 256) hist[0][t] += v;
      __syncthreads();
    }
    if (t < 256) {
      const uint64_t sd = hist[0][t], above = t > 0 ? hist[0][t - 1] : 0ull;  // S[d], S[d + 1]
      const bool reach = strict ? sd > rem : sd >= rem, before = strict ? above > rem : above >= rem;
      if (reach && !before) {
        choice = 255 - t;
        rem_sh = rem - above;
      }
    }
    __syncthreads();
    if (choice < 0) return -1;
    rem = rem_sh;
    prefix |= (uint32_t)choice << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  *found_key = prefix;
  // the ties of that key in id order (the candidates are in id order): each
  // thread a contiguous run, its sum, the prefix over the threads
  const int per = (nc + SNT - 1) / SNT;
  const int c0 = min(nc, t * per), c1 = min(nc, c0 + per);
  uint64_t part = 0;
  for (int c = c0; c < c1; c++)
    if (a.ckey[c] == prefix && k(prefix, a.cid[c])) part += ONE ? 1ull : wfx(a.cp[c], sum);
  uint64_t cum = sblock_exclusive<SNT>(part, shu);
  int hit = INT_MAX;
  for (int c = c0; c < c1; c++) {
    if (a.ckey[c] != prefix || !k(prefix, a.cid[c])) continue;
    cum += ONE ? 1ull : wfx(a.cp[c], sum);
    if (strict ? cum > rem : cum >= rem) {
      hit = a.cid[c];
      break;
    }
  }
  hit = sblock_min<SNT>(hit, shi);
  return hit == INT_MAX ? -1 : hit;
}

// the warpers and the draw over at most SNT candidates sorted in LDS (a
// bitonic sort of key << 32 | ~id, descending: the logit descending, the id
// ascending), each thread one of them: top-k, top-p, min-p and the draw are
// prefixes of that order, their sums a scan in it (sampler.pas:397-449)
__device__ void sorted_pick(const SampleArgs& a, int nc, double sum, uint64_t* sk, double* shd, int* shi)
{
  __shared__ double qh[SNT];
  __shared__ double u_sh2;
  const int t = threadIdx.x;
  sk[t] = t < nc ? ((uint64_t)a.ckey[t] << 32) | (uint64_t)(0xffffffffu - (uint32_t)a.cid[t]) : 0ull;
  for (int k = 2; k <= SNT; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      __syncthreads();
      const int x = t ^ j;
      if (x > t) {
        const uint64_t p = sk[t], q = sk[x];
        if (((t & k) == 0) ? p < q : p > q) {
          sk[t] = q;
          sk[x] = p;
        }
      }
    }
  __syncthreads();
  const uint64_t me = sk[t];
  const uint32_t key = (uint32_t)(me >> 32);
  const int id = (int)(0xffffffffu - (uint32_t)me);
  const double q = t < nc ? a.p[id] / sum : 0.0;
  qh[t] = q;
  // top-k: the first k and every tie of the k-th logit
  int n = nc;
  if (a.top_k > 0 && nc > a.top_k) {
    const uint32_t kk = (uint32_t)(sk[a.top_k - 1] >> 32);
    n = sblock_sum<SNT>((t < nc && key >= kk) ? 1 : 0, shi);
  }
  // the running probability in sorted order over the first n
  double cum = sblock_exclusive<SNT>(t < n ? q : 0.0, shd) + (t < n ? q : 0.0);
  // top-p over what top-k kept: the shortest prefix reaching top_p of its mass
  if (a.top_p < 1.0) {
    double mass = 1.0;
    if (a.top_k > 0) mass = sblock_sum<SNT>(t < n ? q : 0.0, shd);
    const int first = sblock_min<SNT>((t < n && cum >= a.top_p * mass) ? t : INT_MAX, shi);
    if (first != INT_MAX) n = first + 1;
  }
  // min-p: while the probability reaches min_p times the best's
  if (a.min_p > 0.0) {
    const double q0 = qh[0];
    const int fail_at = sblock_min<SNT>((t >= 1 && t < n && !(q >= a.min_p * q0)) ? t : INT_MAX, shi);
    if (fail_at != INT_MAX) n = fail_at;
  }
  // one draw: u times the mass of the first n (the running sum at n - 1),
  // the first whose running sum passes it
  if (t == n - 1) qh[0] = cum;
  __syncthreads();
  if (t == 0) u_sh2 = splitmix_next(a.state) * qh[0];
  __syncthreads();
  const int hit = sblock_min<SNT>((t < n && u_sh2 < cum) ? t : INT_MAX, shi);
  if (t == 0) {
    const int pick = hit == INT_MAX ? 0 : hit;
    *a.out = (int)(0xffffffffu - (uint32_t)sk[pick]);
  }
}

extern "C" __global__ __launch_bounds__(1024) void sample_pick(SampleArgs a)
{
  __shared__ double shd[SNT];
  __shared__ uint64_t shu[SNT];
  __shared__ int shi[SNT];
  __shared__ uint64_t hist[16][256];
  __shared__ double u_sh;
  __shared__ int level, blk;
  __shared__ uint32_t cnt[SBK];
  __shared__ uint64_t mass[SBK];
  const int t = threadIdx.x;
  IHIP_STAMP_SCOPE;
  IHIP_STAMP(0);
  const int best = *a.best;
  __syncthreads();  // every thread has read best before it may be overwritten
  if (sample_greedy(a, best)) {
    if (t == 0) *a.out = best;
    return;
  }
  const double sum = blocks_sum<SNT>(a, shd);
  IHIP_STAMP(1);
  if (!sample_filters(a)) {
    // one draw over every token in id order (sampler.pas:326-342): the block
    // whose running sum passes u, then its tokens
    if (t < a.nb) shd[t] = a.bq[t];
    __syncthreads();
    if (t == 0) {
      const double u = splitmix_next(a.state);
      double cum = 0;
      int bk = -1;
      for (int b = 0; b < a.nb; b++) {
        if (u < cum + shd[b]) {
          bk = b;
          break;
        }
        cum = cum + shd[b];
      }
      blk = bk;
      u_sh = u;
      shd[SNT - 1] = cum;
    }
    __syncthreads();
    const int bk = blk;
    const double u = u_sh, base = shd[SNT - 1];
    __syncthreads();
    int hit = INT_MAX;
    if (bk >= 0) {
      const int per = (a.per + SNT - 1) / SNT;
      const int i0 = min(a.n, bk * a.per + min(a.per, t * per)), i1 = min(min(a.n, (bk + 1) * a.per), i0 + per);
      double part = 0;
      for (int i = i0; i < i1; i++) part = part + a.p[i] / sum;
      double cum = base + sblock_exclusive<SNT>(part, shd);
      for (int i = i0; i < i1; i++) {
        const double q = a.p[i] / sum;
        cum = cum + q;
        if (q > 0 && u < cum) {
          hit = i;
          break;
        }
      }
    }
    hit = sblock_min<SNT>(hit, shi);
    if (t == 0) *a.out = hit == INT_MAX ? best : hit;
    return;
  }
  // the level and the number of candidates (as sample_compact found them)
  bucket_totals<SNT>(a, cnt, mass, shu);
  if (t == 0) {
    const int L = sample_level(a, cnt, mass, sum);
    uint32_t nc = 0;
    for (int k = 0; k <= L; k++) nc += cnt[k];
    level = (int)nc;
  }
  __syncthreads();
  const int nc = level;
  IHIP_STAMP(2);
  if (nc <= SNT) {
    sorted_pick(a, nc, sum, shu, shd, shi);
    return;
  }
  const double qbest = a.p[best] / sum;
  Kept k;
  uint32_t key;
  // top-k: the k-th largest logit; its ties stay (sampler.pas:400-408)
  if (a.top_k > 0 && nc > a.top_k) {
    if (radix_search<true>(a, k, nc, (uint64_t)a.top_k, false, sum, hist, shu, shi, &key) >= 0) k.kmin = key;
  }
  IHIP_STAMP(3);
  // top-p over what top-k kept: the shortest prefix reaching top_p of its
  // mass (sampler.pas:409-428)
  if (a.top_p < 1.0) {
    uint64_t mfx = (uint64_t)FX_ONE;
    if (a.top_k > 0) {
      uint64_t part = 0;
      for (int c = t; c < nc; c += SNT)
        if (k(a.ckey[c], a.cid[c])) part += wfx(a.cp[c], sum);
      mfx = sblock_sum<SNT>(part, shu);
    }
    const uint64_t target = (uint64_t)ceil(a.top_p * (double)mfx);
    const int id = radix_search<false>(a, k, nc, target, false, sum, hist, shu, shi, &key);
    if (id >= 0) {
      k.cut = true;
      k.kp = key;
      k.ip = id;
    }
  }
  IHIP_STAMP(4);
  // min-p, relative to the best token (sampler.pas:429-434): p grows with the
  // logit, so what it keeps is every key from the smallest that passes
  if (a.min_p > 0.0) {
    uint32_t kmin = 0xffffffffu;
    for (int c = t; c < nc; c += SNT)
      if (k(a.ckey[c], a.cid[c]) && a.cp[c] / sum >= a.min_p * qbest) kmin = min(kmin, a.ckey[c]);
    kmin = sblock_min<SNT>(kmin, (uint32_t*)shi);
    k.kmin = max(k.kmin, kmin);
  }
  // one draw from what is left (sampler.pas:435-449)
  uint64_t part = 0;
  for (int c = t; c < nc; c += SNT)
    if (k(a.ckey[c], a.cid[c])) part += wfx(a.cp[c], sum);
  const uint64_t total = sblock_sum<SNT>(part, shu);
  IHIP_STAMP(5);
  if (t == 0) u_sh = splitmix_next(a.state);
  __syncthreads();
  const uint64_t target = (uint64_t)(u_sh * (double)total);
  const int id = radix_search<false>(a, k, nc, target, true, sum, hist, shu, shi, &key);
  IHIP_STAMP(6);
  if (t == 0) *a.out = id >= 0 ? id : best;
}

}  // namespace ihip

// ---------------------------------------------------------- HBM streaming
struct StreamArgs {
  const uint4* p;
  uint64_t n16;
  uint32_t* out;
};

// reads n16 16-byte words once (grid-stride, 8 non-temporal 16-byte loads in
// flight per lane) and folds them so the loads are not dropped: the
// achievable read bandwidth
extern "C" __global__ __launch_bounds__(256) void stream_read(StreamArgs a)
{
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const v4u* p = (const v4u*)a.p;
  for (; i + 7 * stride < a.n16; i += 8 * stride) {
    v4u v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = __builtin_nontemporal_load(p + i + k * stride);
#pragma unroll
    for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < a.n16; i += stride) {
    v4u v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) a.out[0] = acc;
}

// ---------------------------------------------- the next decode step's inputs
// The last launch of a decode step's graph: the step's sampled id becomes the
// next step's token, the position advances, and the next position's rotary
// rows (cos, sin) come from the context's table of positions, so the host
// can enqueue the following steps without waiting for this one.
struct AdvanceArgs {
  const int* next;   // the id this step chose
  int* tok;          // the next step's token
  int* pos;          // the position, advanced by one
  float* cs;         // the rotary row of a position [rs] (cos then sin)
  const float* tab;  // [rows, rs]: the rows of positions 0 .. rows - 1
  float* cs2;        // a second rotary set [rs2], or null
  const float* tab2;
  int32_t rs, rs2, rows, pad;
};
extern "C" __global__ __launch_bounds__(256) void decode_advance(AdvanceArgs a)
{
  const int p = *a.pos + 1;
  if (p < a.rows) {
    for (int i = threadIdx.x; i < a.rs; i += 256) a.cs[i] = a.tab[(int64_t)p * a.rs + i];
    if (a.cs2)
      for (int i = threadIdx.x; i < a.rs2; i += 256) a.cs2[i] = a.tab2[(int64_t)p * a.rs2 + i];
  }
  __syncthreads();  // every read of the position before it moves
  if (threadIdx.x == 0) {
    *a.tok = *a.next;
    *a.pos = p;
  }
}

// ------------------------------------------------------- MoE prompt plan
struct PlanArgs {
  const int* ids;  // [slots] expert of each slot (route, sorted per token)
  int* perm;       // [slots] the slots grouped by expert (any order within one)
  int4* items;     // [max_items] (expert, start in perm, count <= chunk), count 0 after the last
  int32_t slots, experts, max_items, chunk;
};

// the work items of a grouped expert Linear (EnqueueMoe's grouping on the
// device, model.qwen3.cuda.pas:1077-1150): a histogram of the slots per
// expert, a scan for their offsets and for the items' offsets, then every
// slot placed by a counter of its expert. A slot's place within its expert
// changes no output row (each row is its own GEMV/GEMM row), so the counters
// need no order. One block.
extern "C" __global__ __launch_bounds__(256) void moe_plan(PlanArgs a)
{
  __shared__ int cnt[4096], off[4096], fill[4096];
  __shared__ int part[256], ipart[256];
  __shared__ int ntot;
  const int t = threadIdx.x, E = a.experts, S = a.slots, CH = a.chunk;
  for (int e = t; e < E; e += 256) cnt[e] = fill[e] = 0;
  __syncthreads();
  for (int s = t; s < S; s += 256) {
    const int e = a.ids[s];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // thread t owns experts [e0, e1): its sums, scanned over the threads
  const int per = (E + 255) / 256, e0 = min(E, t * per), e1 = min(E, e0 + per);
  int sc = 0, si = 0;
  for (int e = e0; e < e1; e++) {
    sc += cnt[e];
    si += (cnt[e] + CH - 1) / CH;
  }
  part[t] = sc;
  ipart[t] = si;
  __syncthreads();
  if (t == 0) {
    int rs = 0, ri = 0;
    for (int i = 0; i < 256; i++) {
      const int c = part[i], ci = ipart[i];
      part[i] = rs;
      ipart[i] = ri;
      rs += c;
      ri += ci;
    }
    ntot = ri;
  }
  __syncthreads();
  {
    int rs = part[t], ri = ipart[t];
    for (int e = e0; e < e1; e++) {
      off[e] = rs;
      for (int st = 0; st < cnt[e]; st += CH)
        if (ri + st / CH < a.max_items)
          a.items[ri + st / CH] = make_int4(e, rs + st, min(CH, cnt[e] - st), 0);
      rs += cnt[e];
      ri += (cnt[e] + CH - 1) / CH;
    }
  }
  __syncthreads();
  for (int s = t; s < S; s += 256) {
    const int e = a.ids[s];
    if (e >= 0 && e < E) a.perm[off[e] + atomicAdd(&fill[e], 1)] = s;
  }
  for (int it = ntot + t; it < a.max_items; it += 256) a.items[it] = make_int4(0, 0, 0, 0);
}
