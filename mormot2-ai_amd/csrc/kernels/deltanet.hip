// deltanet.hip - the Gated DeltaNet mixer of Qwen3.5 and the output gate of its
// full attention on gfx950: TDecoderModel.DeltaPrep (decoder.pas:2755-2855),
// TInferBackend.DeltaRule (backend.cpu.pas:1890-1972), the gated RMSNorm of
// DeltaNetBlock (decoder.pas:2740-2745) and GateBySigmoid (:2594-2610); the
// device contract of tools/cuda/deltanet.cu (dnconv, dnprep, deltarule,
// gatednorm, splitgate, gatemul).
//
// The arithmetic is the CPU's: single steps round to single, the sums are
// double (products of two singles are exact in double, so an fma is the
// CPU's add of the product). Sums over a wave are reduced in a tree, not in
// the CPU's serial order: the double results differ in the last bits, the
// single results they round to almost never.
//
// The states live on the device per DeltaNet layer: conv [channels, kw - 1]
// (the last inputs, oldest first) and S [value heads, value dim, key dim].
#include "common.h"

using namespace ihip;

// Silu (decoder.pas:2612-2623): x / (1 + exp(-x)) in double, 0 below -100
__device__ __forceinline__ float dn_silu(float x)
{
  const double d = x;
  if (d < -100) return 0.0f;
  return (float)(d / (1.0 + exp(-d)));
}

// 1 / (1 + exp(-x)) in double rounded to single, 0 below -100
__device__ __forceinline__ float dn_sigmoid(float x)
{
  const double d = x;
  if (d < -100) return 0.0f;
  return (float)(1.0 / (1.0 + exp(-d)));
}

// the largest convolution and key dimension handled (a lane keeps
// DN_MAXK / 64 values of a state column)
#define DN_MAXKW 8
#define DN_MAXK 256

struct DnConvArgs {
  float* qkv;        // [rows, channels], convolved and silu'd in place
  const float* w;    // [channels, kw]
  float* conv;       // [channels, kw - 1], moved on
  int32_t rows, channels, kw, pad;
};

// the causal depthwise convolution, one thread per channel over every row in
// order: weight kw - 1 takes the new input, weights 0.. the kept inputs
// (oldest first); then silu
extern "C" __global__ __launch_bounds__(256) void dn_conv(DnConvArgs a)
{
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.channels) return;
  const int k1 = a.kw - 1;
  float st[DN_MAXKW], w[DN_MAXKW];
#pragma unroll
  for (int j = 0; j < DN_MAXKW; j++) {
    st[j] = j < k1 ? a.conv[(int64_t)c * k1 + j] : 0.f;
    w[j] = j < a.kw ? a.w[(int64_t)c * a.kw + j] : 0.f;
  }
  float wl = w[0];
#pragma unroll
  for (int j = 1; j < DN_MAXKW; j++)
    if (j == k1) wl = w[j];
  for (int t = 0; t < a.rows; t++) {
    const int64_t i = (int64_t)t * a.channels + c;
    const float x = a.qkv[i];
    double acc = (double)wl * (double)x;
#pragma unroll
    for (int j = 0; j < DN_MAXKW; j++)
      if (j < k1) acc = __builtin_fma((double)w[j], (double)st[j], acc);
#pragma unroll
    for (int j = 0; j + 1 < DN_MAXKW; j++)
      if (j + 1 < k1) st[j] = st[j + 1];
#pragma unroll
    for (int j = 0; j < DN_MAXKW; j++)
      if (j == k1 - 1) st[j] = x;
    a.qkv[i] = dn_silu((float)acc);
  }
#pragma unroll
  for (int j = 0; j < DN_MAXKW; j++)
    if (j < k1) a.conv[(int64_t)c * k1 + j] = st[j];
}

struct DnPrepArgs {
  float* qkv;          // [rows, channels]: [q heads | k heads | v heads]
  float* beta;         // [rows, vh]: in_proj_b, becomes sigmoid(b)
  float* decay;        // [rows, vh]: in_proj_a, becomes the decay
  float* z;            // [rows, vh * dv]: becomes silu(z)
  const float* dt_bias;  // [vh]
  const float* neg_a;    // [vh]: -exp(A_log)
  int32_t kh, vh, dk, dv, channels, pad;
};

// per (item, row), one wave: a q or k head L2-normed (x / sqrt(sum x^2 +
// 1e-6), the queries also times dk^-0.5 as a single factor); a value head:
// beta = sigmoid(b), decay = exp(neg_a * softplus(a + dt_bias)) (beyond 20
// softplus is its input; below 1e-6 exp gives log1p's value e - e^2 / 2),
// silu of its z
extern "C" __global__ __launch_bounds__(64) void dn_prep(DnPrepArgs a)
{
  const int item = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int i = item - 2 * a.kh;
  if (i < 0) {
    float* s = a.qkv + (int64_t)t * a.channels + (int64_t)item * a.dk;
    double acc = 0;
    for (int j = lane; j < a.dk; j += 64) {
      const double e = s[j];
      acc = __builtin_fma(e, e, acc);
    }
    acc = wave_sum(acc, 64);
    const float f = (float)(1.0 / sqrt(acc + 1e-6));
    const float scale = (float)(1.0 / sqrt((double)a.dk));
    for (int j = lane; j < a.dk; j += 64) {
      float v = s[j] * f;
      if (item < a.kh) v = v * scale;
      s[j] = v;
    }
    return;
  }
  const int64_t f = (int64_t)t * a.vh + i;
  if (lane == 0) {
    a.beta[f] = dn_sigmoid(a.beta[f]);
    const float x = a.decay[f] + a.dt_bias[i];
    float sp;
    if (x > 20) {
      sp = x;
    } else {
      const double e = exp((double)x);
      sp = e < 1e-6 ? (float)(e - e * e / 2) : (float)log(1.0 + e);
    }
    sp = a.neg_a[i] * sp;
    a.decay[f] = (float)exp((double)sp);
  }
  float* zz = a.z + f * a.dv;
  for (int j = lane; j < a.dv; j += 64) zz[j] = dn_silu(zz[j]);
}

struct DnConvPrepArgs {
  float* qkv;          // [channels]: one row, convolved, silu'd and prepared in place
  const float* w;      // [channels, kw]
  float* conv;         // [channels, kw - 1], moved on
  float* beta;         // [vh]
  float* decay;        // [vh]
  float* z;            // [vh * dv]
  const float* dt_bias;
  const float* neg_a;
  int32_t kh, vh, dk, dv, channels, kw;
};

// one row: the convolution of an item's channels and the item's DeltaPrep in
// one launch (dn_conv then dn_prep's arithmetic), one wave per item - a q or
// k head (its dk channels convolved, then L2-normed), or a value head (its dv
// channels convolved; beta, decay, silu(z))
extern "C" __global__ __launch_bounds__(64) void dn_convprep1(DnConvPrepArgs a)
{
  const int item = blockIdx.x, lane = threadIdx.x;
  const int i = item - 2 * a.kh;
  const int first = i < 0 ? item * a.dk : 2 * a.kh * a.dk + i * a.dv;
  const int cnt = i < 0 ? a.dk : a.dv;
  const int k1 = a.kw - 1;
  constexpr int NC = DN_MAXK / 64;  // channels per lane (items of up to 256)
  float y[NC];
#pragma unroll
  for (int u = 0; u < NC; u++) {
    y[u] = 0.f;
    const int cc = lane + 64 * u;
    if (cc >= cnt) continue;
    const int64_t c = first + cc;
    float st[DN_MAXKW], w[DN_MAXKW];
#pragma unroll
    for (int j = 0; j < DN_MAXKW; j++) {
      st[j] = j < k1 ? a.conv[c * k1 + j] : 0.f;
      w[j] = j < a.kw ? a.w[c * a.kw + j] : 0.f;
    }
    float wl = w[0];
#pragma unroll
    for (int j = 1; j < DN_MAXKW; j++)
      if (j == k1) wl = w[j];
    const float x = a.qkv[c];
    double acc = (double)wl * (double)x;
#pragma unroll
    for (int j = 0; j < DN_MAXKW; j++)
      if (j < k1) acc = __builtin_fma((double)w[j], (double)st[j], acc);
#pragma unroll
    for (int j = 0; j + 1 < DN_MAXKW; j++)
      if (j + 1 < k1) a.conv[c * k1 + j] = st[j + 1];
    if (k1 > 0) a.conv[c * k1 + k1 - 1] = x;
    y[u] = dn_silu((float)acc);
  }
  if (i < 0) {
    double acc = 0;
#pragma unroll
    for (int u = 0; u < NC; u++) {
      const double e = y[u];
      acc = __builtin_fma(e, e, acc);
    }
    acc = wave_sum(acc, 64);
    const float f = (float)(1.0 / sqrt(acc + 1e-6));
    const float scale = (float)(1.0 / sqrt((double)a.dk));
#pragma unroll
    for (int u = 0; u < NC; u++) {
      const int cc = lane + 64 * u;
      if (cc >= cnt) continue;
      float v = y[u] * f;
      if (item < a.kh) v = v * scale;
      a.qkv[first + cc] = v;
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < NC; u++) {
    const int cc = lane + 64 * u;
    if (cc < cnt) a.qkv[first + cc] = y[u];
  }
  if (lane == 0) {
    a.beta[i] = dn_sigmoid(a.beta[i]);
    const float x = a.decay[i] + a.dt_bias[i];
    float sp;
    if (x > 20) {
      sp = x;
    } else {
      const double e = exp((double)x);
      sp = e < 1e-6 ? (float)(e - e * e / 2) : (float)log(1.0 + e);
    }
    sp = a.neg_a[i] * sp;
    a.decay[i] = (float)exp((double)sp);
  }
  float* zz = a.z + (int64_t)i * a.dv;
  for (int j = lane; j < a.dv; j += 64) zz[j] = dn_silu(zz[j]);
}

struct DnRuleArgs {
  const float* qkv;    // [rows, stride]: [q heads | k heads | v heads]
  const float* beta;   // [rows, vh]
  const float* decay;  // [rows, vh]
  float* state;        // [vh, dv, dk]
  float* y;            // [rows, vh * dv]
  int32_t rows, stride, kh, vh, dk, dv, group, pad;
};

// the delta rule over rows tokens in order: one wave per column j of a
// value head's S (block = 4 columns of one head), the column in registers
// (DN_MAXK / 64 values per lane) across every token. Per token: the column
// decayed, what it predicts for the key (a double sum), delta = (v_j -
// prediction) * beta, k * delta written in, the column read by the query.
// The next token's operands are loaded while this one is computed.
extern "C" __global__ __launch_bounds__(256) void dn_rule(DnRuleArgs a)
{
  constexpr int NV = DN_MAXK / 64;
  const int head = blockIdx.x, lane = threadIdx.x & 63;
  const int j = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (j >= a.dv) return;
  const int kd = a.kh * a.dk, vdw = a.vh * a.dv;
  const int off = ((head / a.group) % a.kh) * a.dk;
  float* col = a.state + ((int64_t)head * a.dv + j) * a.dk;
  float s[NV];
#pragma unroll
  for (int m = 0; m < NV; m++) {
    const int i = lane + 64 * m;
    s[m] = i < a.dk ? col[i] : 0.f;
  }
  // the operands of token t: q and k of the key head (lane's share), v_j,
  // the decay and beta of the head
  float q[NV], k[NV], v = 0.f, g = 0.f, b = 0.f;
  auto load = [&](int t, float (&qq)[NV], float (&kk)[NV], float& vv, float& gg, float& bb) {
    const float* r = a.qkv + (int64_t)t * a.stride;
#pragma unroll
    for (int m = 0; m < NV; m++) {
      const int i = lane + 64 * m;
      qq[m] = i < a.dk ? r[off + i] : 0.f;
      kk[m] = i < a.dk ? r[kd + off + i] : 0.f;
    }
    vv = r[2 * kd + head * a.dv + j];
    gg = a.decay[(int64_t)t * a.vh + head];
    bb = a.beta[(int64_t)t * a.vh + head];
  };
  if (a.rows > 0) load(0, q, k, v, g, b);
  for (int t = 0; t < a.rows; t++) {
    float qn[NV] = {}, kn[NV] = {}, vn = 0.f, gn = 0.f, bn = 0.f;
    if (t + 1 < a.rows) load(t + 1, qn, kn, vn, gn, bn);
    double acc = 0;
#pragma unroll
    for (int m = 0; m < NV; m++) {
      s[m] = s[m] * g;
      acc = __builtin_fma((double)s[m], (double)k[m], acc);
    }
    acc = wave_sum(acc, 64);
    const float pred = (float)acc;
    float delta = v - pred;
    delta = delta * b;
    double o = 0;
#pragma unroll
    for (int m = 0; m < NV; m++) {
      const float p = k[m] * delta;
      s[m] = s[m] + p;
      o = __builtin_fma((double)s[m], (double)q[m], o);
    }
    o = wave_sum(o, 64);
    if (lane == 0) a.y[(int64_t)t * vdw + head * a.dv + j] = (float)o;
#pragma unroll
    for (int m = 0; m < NV; m++) {
      q[m] = qn[m];
      k[m] = kn[m];
    }
    v = vn;
    g = gn;
    b = bn;
  }
#pragma unroll
  for (int m = 0; m < NV; m++) {
    const int i = lane + 64 * m;
    if (i < a.dk) col[i] = s[m];
  }
}

struct DnNormArgs {
  float* x;        // [rows, cols]: the rule's output, normed and gated in place
  const float* w;  // [cols]
  const float* z;  // [rows, cols]: silu(z)
  double eps;
  int32_t rows, cols;
};

// the gated RMSNorm of every value head's output, one wave per row: the
// RMSNorm of TInferCpuBackend.RmsNorm (double sum, x * inv rounded to single
// before the weight), then times silu(z)
extern "C" __global__ __launch_bounds__(256) void dn_gatenorm(DnNormArgs a)
{
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.rows) return;
  float* x = a.x + (int64_t)row * a.cols;
  const float* z = a.z + (int64_t)row * a.cols;
  double s = 0;
  for (int c = lane; c < a.cols; c += 64) {
    const double d = x[c];
    s = __builtin_fma(d, d, s);
  }
  s = wave_sum(s, 64);
  const double inv = 1.0 / sqrt(s / (double)a.cols + a.eps);
  for (int c = lane; c < a.cols; c += 64) {
    const float n = (float)((double)x[c] * inv);
    const float y = a.w[c] * n;
    x[c] = y * z[c];
  }
}

struct GateArgs {
  const float* qg;  // split_gate: [rows * heads, 2 * hd]
  float* q;         // split_gate: [rows * heads, hd]; gate_sigmoid: the attention output
  float* g;         // [rows * heads, hd]: the gates
  int64_t n;        // rows * heads * hd
  int32_t hd, pad;
};

// the query projection of a gated attention holds per head its query, then
// its gate: apart into q and g
extern "C" __global__ __launch_bounds__(256) void split_gate(GateArgs a)
{
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  const int64_t r = i / a.hd, c = i - r * a.hd;
  a.q[i] = a.qg[r * 2 * a.hd + c];
  a.g[i] = a.qg[r * 2 * a.hd + a.hd + c];
}

// GateBySigmoid: q[i] *= sigmoid(g[i]), the sigmoid rounded to single first
extern "C" __global__ __launch_bounds__(256) void gate_sigmoid(GateArgs a)
{
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  a.q[i] = a.q[i] * dn_sigmoid(a.g[i]);
}
