// ops.hip - the operations of a decoder layer besides Linear, for gfx950.
//
// Each kernel follows the arithmetic of the reference's CPU backend
// (src/infer/mormot.ai.infer.backend.cpu.pas) step by step - double sums
// where the CPU sums in double, single roundings where it rounds - so that a
// forward pass on the device gives the CPU's logits up to the order of
// double sums. Sums across lanes run as wave/block reductions.
#include "common.h"

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
  for (int o = 1; o < 64; o <<= 1) {
    float oa = __shfl_xor(amax, o), om = __shfl_xor(m, o);
    int oi = __shfl_xor(idx, o);
    if (oa > amax || (oa == amax && oi < idx)) {
      amax = oa;
      m = om;
      idx = oi;
    }
  }
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
};

// TInferCpuBackend.RmsNorm (backend.cpu.pas:1769-1795): the sum of squares in
// double, inv = 1 / sqrt(mean + eps) in double, x * inv rounded to single
// before the weight; with t: x += t first (addnorm, ops.cu:135-150)
extern "C" __global__ __launch_bounds__(256) void rmsnorm(NormArgs a)
{
  __shared__ double sh[4];
  int64_t base = (int64_t)blockIdx.x * a.cols;
  double s = 0;
  for (int c = threadIdx.x; c < a.cols; c += blockDim.x) {
    float v = a.x[base + c];
    if (a.t) {
      v = v + a.t[base + c];
      a.x[base + c] = v;
    }
    double d = v;
    s = s + d * d;
  }
  s = block_sum_d(s, sh);
  double inv = 1.0 / sqrt(s / (double)a.cols + a.eps);
  for (int c = threadIdx.x; c < a.cols; c += blockDim.x) {
    float n = (float)((double)a.x[base + c] * inv);
    a.y[base + c] = a.w[c] * n;
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

// ------------------------------------------------------------------ qkrope
struct RopeArgs {
  float* q;
  const float* k;
  const float* v;
  const float* qn;  // [hd] or null: no per-head norm
  const float* kn;
  const float* cs;  // [rows, hd/2] cos, then [rows, hd/2] sin
  void* kc;         // cache [*, kvh * hd] float or half
  void* vc;
  const int* pastp;  // device position of row 0 (graph replay), or null: past
  double eps;
  int32_t rows, heads, kvh, hd, past, f16;
};

// per (head: the q heads, then the kv heads; row): the Q/K head RMSNorm of
// decoder.pas:2668-2673, rotate_half RoPE in double (backend.cpu.pas:
// 1862-1888), K and V stored into the cache at past + row (decoder.pas:
// 2688-2691); one wave per head
extern "C" __global__ __launch_bounds__(64) void qkrope(RopeArgs a)
{
  __shared__ float nv[512];
  int hh = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  int d = a.hd, half = d >> 1;
  const int past = a.pastp ? *a.pastp : a.past;
  bool isq = hh < a.heads;
  int h = isq ? hh : hh - a.heads;
  int64_t src = isq ? ((int64_t)r * a.heads + h) * d : ((int64_t)r * a.kvh + h) * d;
  const float* in = isq ? a.q + src : a.k + src;
  const float* nw = isq ? a.qn : a.kn;
  if (nw) {
    double s = 0;
    for (int c = t; c < d; c += 64) {
      double x = in[c];
      s = s + x * x;
    }
    s = wave_sum(s, 64);
    double inv = 1.0 / sqrt(s / (double)d + a.eps);
    for (int c = t; c < d; c += 64) {
      float n = (float)((double)in[c] * inv);
      nv[c] = nw[c] * n;
    }
  } else {
    for (int c = t; c < d; c += 64) nv[c] = in[c];
  }
  __syncthreads();
  const float* cr = a.cs + (int64_t)r * half;
  const float* sr = a.cs + (int64_t)a.rows * half + (int64_t)r * half;
  int64_t kvw = (int64_t)a.kvh * d;
  int64_t dst = ((int64_t)past + r) * kvw + (int64_t)h * d;
  for (int i = t; i < half; i += 64) {
    double x0 = nv[i], x1 = nv[i + half], c = cr[i], s = sr[i];
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
  if (!isq)
    for (int c = t; c < d; c += 64) {
      float vv = a.v[src + c];
      if (a.f16) ((uint16_t*)a.vc)[dst + c] = float_to_half(vv);
      else ((float*)a.vc)[dst + c] = vv;
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
  double scale;
  int32_t rows, heads, kvh, hd, past, window, f16, maxkeys;
};

__device__ __forceinline__ double cache_at(const void* c, int64_t i, int f16)
{
  return f16 ? (double)half_to_float(((const uint16_t*)c)[i]) : (double)((const float*)c)[i];
}

// the reference rows of CausalRows (backend.cpu.pas:1305-1354): each score a
// sequential double dot product (the CPU's bits), the maximum and the sink
// taken out, exp in double, the weighted values summed in double, divided at
// the end. One block of 256 per (head, row); the scores of the keys live in
// LDS (maxkeys doubles, checked by the host).
extern "C" __global__ __launch_bounds__(256) void attention(AttnArgs a)
{
  extern __shared__ double sc[];
  __shared__ double red[8];
  __shared__ double part[256];
  int h = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  int d = a.hd;
  int64_t kvw = (int64_t)a.kvh * d, qw = (int64_t)a.heads * d;
  int g = h / (a.heads / a.kvh);
  const int past = a.pastp ? *a.pastp : a.past;
  int total = past + r + 1, first = 0;
  if (a.window > 0 && total > a.window) first = total - a.window;
  int cnt = total - first;
  const float* q = a.q + (int64_t)r * qw + (int64_t)h * d;
  double mloc = -1.0e308;
  for (int j = t; j < cnt; j += blockDim.x) {
    int64_t kb = (int64_t)(first + j) * kvw + (int64_t)g * d;
    double acc = 0;
    for (int i = 0; i < d; i++) acc = acc + (double)q[i] * cache_at(a.kc, kb + i, a.f16);
    acc = acc * a.scale;
    sc[j] = acc;
    if (acc > mloc) mloc = acc;
  }
  // the maximum of the block
  for (int o = 1; o < 64; o <<= 1) {
    double ov = __shfl_xor(mloc, o);
    if (ov > mloc) mloc = ov;
  }
  if ((t & 63) == 0) red[t >> 6] = mloc;
  __syncthreads();
  double m = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); i++)
    if (red[i] > m) m = red[i];
  if (a.sinks && (double)a.sinks[h] > m) m = a.sinks[h];
  double s = 0;
  for (int j = t; j < cnt; j += blockDim.x) {
    double e = exp(sc[j] - m);
    sc[j] = e;
    s = s + e;
  }
  __syncthreads();
  s = wave_sum(s, 64);
  if ((t & 63) == 0) red[4 + (t >> 6)] = s;
  __syncthreads();
  double sum = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) sum = sum + red[4 + i];
  if (a.sinks) sum = sum + exp((double)a.sinks[h] - m);
  // the weighted values: thread t sums dimension t % d over its key share
  int nsplit = blockDim.x / d;  // hd 64: 4, hd 128: 2, hd 256: 1
  int dim = t % d, sp = t / d;
  double acc = 0;
  if (sp < nsplit) {
    int per = (cnt + nsplit - 1) / nsplit;
    int j0 = sp * per, j1 = min(cnt, j0 + per);
    for (int j = j0; j < j1; j++)
      acc = acc + sc[j] * cache_at(a.vc, (int64_t)(first + j) * kvw + (int64_t)g * d + dim, a.f16);
  }
  part[t] = acc;
  __syncthreads();
  if (t < d) {
    double tot = part[t];
    for (int i = 1; i < nsplit; i++) tot = tot + part[i * d + t];
    a.y[(int64_t)r * qw + (int64_t)h * d + t] = (float)(tot * (1.0 / sum));
  }
}

// ------------------------------------------------------------------- MoE
struct RouteArgs {
  const float* logits;
  int* ids;
  float* w;
  int32_t experts, k, norm, rows;
};

// TDecoderModel.Route (decoder.pas:2901-2949) = route of ops.cu:664-720:
// softmax in double, the k highest logits (lower id on a tie), weights
// rounded to single, renormed, then sorted by id; one thread per row
extern "C" __global__ __launch_bounds__(64) void route(RouteArgs a)
{
  int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= a.rows) return;
  const float* lg = a.logits + (int64_t)row * a.experts;
  uint32_t taken[128];
  int chosen[64];
  float wt[64];
  for (int i = 0; i < 128; i++) taken[i] = 0;
  double m = lg[0];
  for (int i = 1; i < a.experts; i++)
    if (lg[i] > m) m = lg[i];
  double sum = 0;
  for (int i = 0; i < a.experts; i++) sum = sum + exp((double)lg[i] - m);
  double picked = 0;
  for (int j = 0; j < a.k; j++) {
    int best = -1;
    for (int i = 0; i < a.experts; i++)
      if (((taken[i >> 5] >> (i & 31)) & 1u) == 0u && (best < 0 || lg[i] > lg[best])) best = i;
    taken[best >> 5] |= 1u << (best & 31);
    chosen[j] = best;
    wt[j] = (float)(exp((double)lg[best] - m) / sum);
    picked = picked + (double)wt[j];
  }
  if (a.norm)
    for (int j = 0; j < a.k; j++) wt[j] = (float)((double)wt[j] / picked);
  for (int j = 1; j < a.k; j++) {
    int id = chosen[j];
    float v = wt[j];
    int p = j;
    while (p > 0 && chosen[p - 1] > id) {
      chosen[p] = chosen[p - 1];
      wt[p] = wt[p - 1];
      p--;
    }
    chosen[p] = id;
    wt[p] = v;
  }
  for (int j = 0; j < a.k; j++) {
    a.ids[(int64_t)row * a.k + j] = chosen[j];
    a.w[(int64_t)row * a.k + j] = wt[j];
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
};

// InferArgMax (sampler.pas:123-160): the float bits ordered as integers (the
// lower 31 flipped when negative, -0 as +0), NaN skipped, the first index of
// the maximum; all NaN gives 0. One block of 1024.
extern "C" __global__ __launch_bounds__(1024) void argmax(ArgmaxArgs a)
{
  __shared__ int bk[16];
  __shared__ int64_t bi[16];
  int best = INT32_MIN;
  int64_t bidx = INT64_MAX;
  for (int64_t i = threadIdx.x; i < a.n; i += blockDim.x) {
    uint32_t b = float_bits(a.v[i]);
    if ((b & 0x7fffffffu) > 0x7f800000u) continue;
    int k = (int)(b ^ ((b >> 31) * 0x7fffffffu));
    if (k == -1) k = 0;
    if (k > best) {
      best = k;
      bidx = i;
    }
  }
  for (int o = 1; o < 64; o <<= 1) {
    int ok = __shfl_xor(best, o);
    int64_t oi = __shfl_xor(bidx, o);
    if (ok > best || (ok == best && oi < bidx)) {
      best = ok;
      bidx = oi;
    }
  }
  int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bk[w] = best;
    bi[w] = bidx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int b = bk[0];
    int64_t ix = bi[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++)
      if (bk[i] > b || (bk[i] == b && bi[i] < ix)) {
        b = bk[i];
        ix = bi[i];
      }
    a.out[0] = ix == INT64_MAX ? 0 : (int)ix;
  }
}

}  // namespace ihip

// ---------------------------------------------------------- HBM streaming
struct StreamArgs {
  const uint4* p;
  uint64_t n16;
  uint32_t* out;
};

// reads n16 16-byte words once (grid-stride, 4 in flight per lane) and folds
// them so the loads are not dropped: the achievable read bandwidth
extern "C" __global__ __launch_bounds__(256) void stream_read(StreamArgs a)
{
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < a.n16; i += 4 * stride) {
    uint4 v0 = a.p[i], v1 = a.p[i + stride], v2 = a.p[i + 2 * stride], v3 = a.p[i + 3 * stride];
    acc ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
    acc ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
  }
  for (; i < a.n16; i += stride) {
    uint4 v = a.p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) a.out[0] = acc;
}

// ------------------------------------------------------- MoE prompt plan
struct PlanArgs {
  const int* ids;  // [slots] expert of each slot (route, sorted per token)
  int* perm;       // [slots] the slots sorted by expert, in slot order within one
  int4* items;     // [max_items] (expert, start in perm, count <= 8), count 0 after the last
  int32_t slots, experts, max_items, pad;
};

// the experts of a prompt chunk grouped for the batched GEMV (the host-side
// expert loop of model.qwen3.cuda.pas:1077-1150, on the device): a count per
// expert, their offsets, then per expert its slots in order - thread e
// collects expert e, so the order is deterministic
extern "C" __global__ __launch_bounds__(256) void moe_plan(PlanArgs a)
{
  __shared__ int cnt[4096];
  __shared__ int off[4096];
  __shared__ int sid[4096];
  const int t = threadIdx.x, E = a.experts, S = a.slots;
  for (int e = t; e < E; e += blockDim.x) cnt[e] = 0;
  for (int s = t; s < S; s += blockDim.x) sid[s] = a.ids[s];
  __syncthreads();
  for (int s = t; s < S; s += blockDim.x) {
    int e = sid[s];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (t == 0) {
    int run = 0, it = 0;
    for (int e = 0; e < E; e++) {
      off[e] = run;
      for (int st = 0; st < cnt[e] && it < a.max_items; st += 8)
        a.items[it++] = make_int4(e, run + st, min(8, cnt[e] - st), 0);
      run += cnt[e];
    }
    for (; it < a.max_items; it++) a.items[it] = make_int4(0, 0, 0, 0);
  }
  __syncthreads();
  for (int e = t; e < E; e += blockDim.x) {
    int k = off[e];
    for (int s = 0; s < S; s++)
      if (sid[s] == e) a.perm[k++] = s;
  }
}
