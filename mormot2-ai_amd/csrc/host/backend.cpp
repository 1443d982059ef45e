// backend.cpp - TInferCudaBackend of the reference
// (src/infer/mormot.ai.infer.backend.cuda.pas:51-517) for HIP: the weight
// cache with its repack into the HIP layout, the Linear dispatch (GEMV kernel
// per dtype, arithmetic and shape), and the enqueue wrappers of the layer
// operations.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <thread>

#include "internal.h"

namespace ihip {

// ---------------------------------------------------------------- repack
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// the value i (0..255) of a GGUF Q6_K super-block, 0..63 (Q6KValue + 32,
// tensor.pas:419-439)
static inline int q6_value(const uint8_t* b, int i)
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
  return r | (h << 4);
}

// one row o of matrix m: GGUF blocks at src -> regions of dst (base of the matrix)
static void repack_row(const uint8_t* src, uint8_t* dst, int t, int64_t out, int64_t in, int64_t o)
{
  const Regions rg = regions(t, out, in);
  const int64_t G = in / 32, NB = in / 256;
  switch (t) {
  case DT_Q8_0:
    for (int64_t b = 0; b < G; b++) {
      const uint8_t* s = src + b * 34;
      memcpy(dst + rg.s + (o * G + b) * 2, s, 2);
      memcpy(dst + o * in + b * 16, s + 2, 16);
      memcpy(dst + o * in + in / 2 + b * 16, s + 18, 16);
    }
    break;
  case DT_Q4_0:
    for (int64_t b = 0; b < G; b++) {
      const uint8_t* s = src + b * 18;
      memcpy(dst + rg.s + (o * G + b) * 2, s, 2);
      memcpy(dst + (o * G + b) * 16, s + 2, 16);
    }
    break;
  case DT_MXFP4:
    for (int64_t b = 0; b < G; b++) {
      const uint8_t* s = src + b * 17;
      dst[rg.s + o * G + b] = s[0];
      memcpy(dst + (o * G + b) * 16, s + 1, 16);
    }
    break;
  case DT_Q5_0:
    for (int64_t b = 0; b < G; b++) {
      const uint8_t* s = src + b * 22;
      memcpy(dst + rg.s + (o * G + b) * 2, s, 2);
      memcpy(dst + rg.h + (o * G + b) * 4, s + 2, 4);
      memcpy(dst + (o * G + b) * 16, s + 6, 16);
    }
    break;
  case DT_Q5_1:
    for (int64_t b = 0; b < G; b++) {
      const uint8_t* s = src + b * 24;
      memcpy(dst + rg.s + (o * G + b) * 4, s, 4);
      memcpy(dst + rg.h + (o * G + b) * 4, s + 4, 4);
      memcpy(dst + (o * G + b) * 16, s + 8, 16);
    }
    break;
  case DT_Q4_K:
    for (int64_t b = 0; b < NB; b++) {
      const uint8_t* s = src + b * 144;
      memcpy(dst + rg.s + (o * NB + b) * 16, s, 16);
      const uint8_t* qs = s + 16;
      for (int jj = 0; jj < 8; jj++) {
        uint8_t* gq = dst + (o * G + b * 8 + jj) * 16;
        int k = jj >> 1, sh = (jj & 1) * 4;
        for (int j = 0; j < 16; j++) {
          int lo = (qs[32 * k + j] >> sh) & 15, hi = (qs[32 * k + j + 16] >> sh) & 15;
          gq[j] = (uint8_t)(lo | (hi << 4));
        }
      }
    }
    break;
  case DT_Q6_K:
    for (int64_t b = 0; b < NB; b++) {
      const uint8_t* s = src + b * 210;
      memcpy(dst + rg.s + (o * NB + b) * 16, s + 192, 16);
      memcpy(dst + rg.s2 + (o * NB + b) * 2, s + 208, 2);
      for (int u = 0; u < 8; u++) {
        uint8_t* gq = dst + (o * G + b * 8 + u) * 16;
        uint8_t* gh = dst + rg.h + (o * G + b * 8 + u) * 8;
        memset(gh, 0, 8);
        for (int j = 0; j < 16; j++) {
          int lo = q6_value(s, 32 * u + j), hi = q6_value(s, 32 * u + j + 16);
          gq[j] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
          int d = j >> 2, i = j & 3;
          gh[i] |= (uint8_t)((lo >> 4) << (2 * d));
          gh[4 + i] |= (uint8_t)((hi >> 4) << (2 * d));
        }
      }
    }
    break;
  default:  // float types: unchanged
    memcpy(dst + o * (int64_t)row_bytes(t, in), src, row_bytes(t, in));
    break;
  }
}

static void unpack_row(const uint8_t* src, uint8_t* dst, int t, int64_t out, int64_t in, int64_t o)
{
  const Regions rg = regions(t, out, in);
  const int64_t G = in / 32, NB = in / 256;
  switch (t) {
  case DT_Q8_0:
    for (int64_t b = 0; b < G; b++) {
      memcpy(dst + b * 34, src + rg.s + (o * G + b) * 2, 2);
      memcpy(dst + b * 34 + 2, src + o * in + b * 16, 16);
      memcpy(dst + b * 34 + 18, src + o * in + in / 2 + b * 16, 16);
    }
    break;
  case DT_Q4_0:
    for (int64_t b = 0; b < G; b++) {
      memcpy(dst + b * 18, src + rg.s + (o * G + b) * 2, 2);
      memcpy(dst + b * 18 + 2, src + (o * G + b) * 16, 16);
    }
    break;
  case DT_MXFP4:
    for (int64_t b = 0; b < G; b++) {
      dst[b * 17] = src[rg.s + o * G + b];
      memcpy(dst + b * 17 + 1, src + (o * G + b) * 16, 16);
    }
    break;
  case DT_Q5_0:
    for (int64_t b = 0; b < G; b++) {
      memcpy(dst + b * 22, src + rg.s + (o * G + b) * 2, 2);
      memcpy(dst + b * 22 + 2, src + rg.h + (o * G + b) * 4, 4);
      memcpy(dst + b * 22 + 6, src + (o * G + b) * 16, 16);
    }
    break;
  case DT_Q5_1:
    for (int64_t b = 0; b < G; b++) {
      memcpy(dst + b * 24, src + rg.s + (o * G + b) * 4, 4);
      memcpy(dst + b * 24 + 4, src + rg.h + (o * G + b) * 4, 4);
      memcpy(dst + b * 24 + 8, src + (o * G + b) * 16, 16);
    }
    break;
  case DT_Q4_K:
    for (int64_t b = 0; b < NB; b++) {
      uint8_t* d = dst + b * 144;
      memcpy(d, src + rg.s + (o * NB + b) * 16, 16);
      memset(d + 16, 0, 128);
      for (int jj = 0; jj < 8; jj++) {
        const uint8_t* gq = src + (o * G + b * 8 + jj) * 16;
        int k = jj >> 1, sh = (jj & 1) * 4;
        for (int j = 0; j < 16; j++) {
          d[16 + 32 * k + j] |= (uint8_t)((gq[j] & 15) << sh);
          d[16 + 32 * k + j + 16] |= (uint8_t)((gq[j] >> 4) << sh);
        }
      }
    }
    break;
  case DT_Q6_K:
    for (int64_t b = 0; b < NB; b++) {
      uint8_t* d = dst + b * 210;
      memset(d, 0, 192);
      memcpy(d + 192, src + rg.s + (o * NB + b) * 16, 16);
      memcpy(d + 208, src + rg.s2 + (o * NB + b) * 2, 2);
      for (int u = 0; u < 8; u++) {
        const uint8_t* gq = src + (o * G + b * 8 + u) * 16;
        const uint8_t* gh = src + rg.h + (o * G + b * 8 + u) * 8;
        for (int v = 0; v < 32; v++) {
          int j = v & 15, hiv = v >> 4, dd = j >> 2, ii = j & 3;
          int q = (hiv ? (gq[j] >> 4) : (gq[j] & 15)) | (((gh[4 * hiv + ii] >> (2 * dd)) & 3) << 4);
          int i = 32 * u + v, n = i >> 7, l = i & 31, qq = (i & 127) >> 5;
          d[128 + 32 * n + l] |= (uint8_t)((q >> 4) << (2 * qq));
          int qi = 64 * n + l + ((qq & 1) ? 32 : 0);
          d[qi] |= (uint8_t)((q & 15) << (qq >= 2 ? 4 : 0));
        }
      }
    }
    break;
  default:
    memcpy(dst, src + o * (int64_t)row_bytes(t, in), row_bytes(t, in));
    break;
  }
}

static void for_rows(int64_t total, const std::function<void(int64_t, int64_t)>& fn)
{
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (total < 4096 || nt == 1) {
    fn(0, total);
    return;
  }
  std::vector<std::thread> th;
  int64_t per = (total + nt - 1) / nt;
  for (unsigned i = 0; i < nt; i++) {
    int64_t a = i * per, b = std::min(total, a + per);
    if (a < b) th.emplace_back(fn, a, b);
  }
  for (auto& x : th) x.join();
}

void repack(const void* src, void* dst, int t, int64_t out, int64_t in, int64_t count)
{
  const uint64_t rb = row_bytes(t, in), mb = rb * out;
  for_rows(count * out, [&](int64_t a, int64_t b) {
    for (int64_t i = a; i < b; i++) {
      int64_t m = i / out, o = i % out;
      repack_row((const uint8_t*)src + m * mb + o * rb, (uint8_t*)dst + m * mb, t, out, in, o);
    }
  });
}

void unpack(const void* src, void* dst, int t, int64_t out, int64_t in, int64_t count)
{
  const uint64_t rb = row_bytes(t, in), mb = rb * out;
  for_rows(count * out, [&](int64_t a, int64_t b) {
    for (int64_t i = a; i < b; i++) {
      int64_t m = i / out, o = i % out;
      unpack_row((const uint8_t*)src + m * mb, (uint8_t*)dst + m * mb + o * rb, t, out, in, o);
    }
  });
}

// --------------------------------------------------------------- dispatch
static const char* fmt_name(int t)
{
  switch (t) {
  case DT_Q8_0: return "q8_0";
  case DT_Q4_0: return "q4_0";
  case DT_MXFP4: return "mxfp4";
  case DT_Q5_0: return "q5_0";
  case DT_Q5_1: return "q5_1";
  case DT_Q4_K: return "q4_k";
  case DT_Q6_K: return "q6_k";
  case DT_F32: return "f32";
  case DT_BF16: return "bf16";
  case DT_F16: return "f16";
  default: return nullptr;
  }
}

int q8_kind(int t)
{
  if (t == DT_Q4_K || t == DT_Q6_K) return 1;
  if (t == DT_F32 || t == DT_BF16 || t == DT_F16) return -1;
  return 0;
}

bool linear_ok(int t, int64_t in)
{
  if (!fmt_name(t) || in <= 0 || in % 32) return false;
  if ((t == DT_Q4_K || t == DT_Q6_K) && in % 256) return false;
  return in / 32 <= 256;  // the activation of a lane's groups stays in registers
}

// lanes per row and groups per lane, the least idle lanes first. Between
// equal choices: narrow rows (more groups per lane: a row's lane sums and its
// addressing are paid once per U groups) when the matrix still gives every CU
// four tiles of them, else wide rows (more waves for a short matrix)
static void pick_lpr_order(int64_t G, const int (&order)[4], int& lpr, int& U, int ulimit = 4)
{
  // at most this many groups per lane (IHIP_GEMV_UMAX, 1..4: fewer give
  // wider rows, shorter per-lane work, more waves)
  static const int umax_env = [] {
    const char* v = getenv("IHIP_GEMV_UMAX");
    return v ? std::min(4, std::max(1, atoi(v))) : 4;
  }();
  const int umax = std::min(umax_env, ulimit);
  int best = -1;
  for (int l : order) {
    int u = (int)((G + l - 1) / l);
    if (u > umax && !(l == 64 && u <= 4)) continue;
    int waste = l * u - (int)G;
    if (best < 0 || waste < best) {
      best = waste;
      lpr = l;
      U = u;
    }
  }
}

static const int glu_order[4] = {8, 16, 32, 64};

static void pick_lpr(int64_t G, int64_t out, int cus, int& lpr, int& U)
{
  static const int narrow_first[4] = {8, 16, 32, 64}, wide_first[4] = {64, 32, 16, 8};
  pick_lpr_order(G, narrow_first, lpr, U);
  if (out / (64 / lpr) < 4 * (int64_t)cus) pick_lpr_order(G, wide_first, lpr, U);
}

uint64_t q8_row_bytes(int64_t in) { return (uint64_t)in + 4 * (uint64_t)(in / 32); }

// bytes of one row staged by gemv_rows (codes, scales, half sums; 16-aligned)
static int rows_stride(int in) { return ((in + 12 * (in / 32)) + 15) & ~15; }

int enqueue_quantize(ihip_ctx* c, uint64_t x, int64_t rows, int64_t in, int kind, uint64_t xq)
{
  struct {
    const float* x;
    uint8_t* xq;
    int* bad;
    int32_t rows, in;
  } a = {(const float*)x, (uint8_t*)xq, (int*)c->scratch_bad, (int32_t)rows, (int32_t)in};
  if (kind == 0) {
    int64_t G = in / 32;
    return launch(c, "quantize_q8_0", dim3((unsigned)((G + 255) / 256), (unsigned)rows), dim3(256), &a);
  }
  int64_t NB = in / 256;
  return launch(c, "quantize_q8_k", dim3((unsigned)((NB + 3) / 4), (unsigned)rows), dim3(256), &a);
}

// weight types of gemm.hip
static bool gemm_fmt(int t)
{
  return t == DT_Q8_0 || t == DT_Q4_0 || t == DT_MXFP4 || t == DT_Q5_0 || t == DT_Q5_1 ||
         t == DT_Q4_K || t == DT_Q6_K || t == DT_F32 || t == DT_BF16 || t == DT_F16;
}

static bool float_fmt(int t) { return t == DT_F32 || t == DT_BF16 || t == DT_F16; }

bool gemv_pair(ihip_ctx* c, int a, int b, int mode, int64_t in)
{
  if (!linear_ok(a, in) || !linear_ok(b, in)) return false;
  int lpr = 64, U = 1;
  pick_lpr(in / 32, 1 << 30, 256, lpr, U);  // the name only: every U has a pair kernel
  char name[64];
  snprintf(name, sizeof name, "gemv_%s_%s_%s_norm_u%d", fmt_name(a), fmt_name(b),
           (mode & 1) == IHIP_MODE_Q8 ? "q8" : "f32", U);
  return kernel(c, name) != nullptr;
}

bool gemm_runs(const ihip_ctx* c, int dtype, int mode)
{
  return c->use_gemm && (mode & 1) == IHIP_MODE_Q8 && gemm_fmt(dtype);
}

int enqueue_linear(ihip_ctx* c, const LinearCall& k)
{
  if (!linear_ok(k.dtype, k.in) || k.out < 1 || k.out > INT32_MAX || k.rows < 1 || k.rows > 65535 ||
      !k.w || !k.x || !k.y)
    return fail(IHIP_E_ARG, "EnqueueLinear: " + std::to_string(k.rows) + " rows of " +
                                std::to_string(k.in) + " dtype " + std::to_string(k.dtype) +
                                " into " + std::to_string(k.out));
  const int64_t G = k.in / 32;
  int lpr = 64, U = 1;
  int64_t out_max = k.out;
  for (int i = 0; i < k.nseg && i < 3; i++) out_max = std::max<int64_t>(out_max, k.oseg[i]);
  // the experts of one token's slots share the launch: their rows together
  // decide between narrow and wide rows
  if (k.ids && !k.cw && !k.items) out_max *= std::max<int64_t>(1, k.rows);
  pick_lpr(G, out_max, c->cus, lpr, U);
  // a token's experts through the fused gate/up: at most 2 groups a lane (rows
  // of more lanes, twice the blocks of 4 groups a lane, each with half the
  // bytes: measured faster for these short matrices)
  if (k.w2 && k.ids && !k.items && U > 2) {
    int l2 = lpr, u2 = U;
    pick_lpr_order(G, glu_order, l2, u2, 2);
    if ((int64_t)l2 * u2 == G) {  // (when no lane idles for it)
      lpr = l2;
      U = u2;
    }
  }
  uint64_t xq = k.xq;
  const int mode = k.mode & 1;
  const bool q8 = mode == IHIP_MODE_Q8 && q8_kind(k.dtype) >= 0;
  if (q8 && (k.mode & IHIP_MODE_XQ)) xq = k.x;  // x is already quantized
  const bool batch = k.items || (!k.ids && k.rows > 1);
  // one activation row per block (decode, experts of a token): the GEMV
  // quantizes its own groups in registers, no separate launch
  if (q8 && !xq && batch) {
    int64_t xrows = (k.ids || k.items)
                        ? (k.x_per_slot ? (k.rows + k.x_per_slot - 1) / k.x_per_slot : 1)
                        : k.rows;
    int rc = scratch(c, c->scratch_q, c->scratch_q_bytes, xrows * q8_row_bytes(k.in));
    if (rc) return rc;
    xq = c->scratch_q;
    rc = enqueue_quantize(c, k.x, xrows, k.in, q8_kind(k.dtype), xq);
    if (rc) return rc;
  }
  struct {
    const uint8_t* w;
    const float* x;
    const uint8_t* xq;
    const float* bias;
    float* y;
    const int* ids;
    int64_t stride;
    int32_t out, in, rows, lpr;
    int32_t x_per_slot;
    int32_t nexp;
    const void* items;
    const int* perm;
    const uint8_t* w2;
    const float* bias2;
    float alpha, limit;
    int* bad;
    const float* nw;
    double eps;
    const float* res;
    const float* cw;
    int32_t kslots;
    int32_t nseg;
    const uint8_t* wseg[3];
    const float* bseg[3];
    float* yseg[3];
    int32_t oseg[3];
    int32_t nseg1;
    const float* rl;
    float* rw;
    int32_t rexp, rk, rnorm, rpad;
    const float* rscale;
    uint8_t* xq_out;
    int32_t xq_k8, xq_pad;
    int32_t bstart[4];
  } a = {(const uint8_t*)k.w, (const float*)k.x, (const uint8_t*)xq, (const float*)k.bias,
         (float*)k.y, (const int*)k.ids, k.stride, (int32_t)k.out, (int32_t)k.in,
         (int32_t)k.rows, lpr, k.x_per_slot, k.nexp, (const void*)k.items, (const int*)k.perm,
         (const uint8_t*)k.w2, (const float*)k.bias2, k.alpha, k.limit, (int*)c->scratch_bad,
         (const float*)k.nw, k.eps, (const float*)k.res, (const float*)k.cw,
         k.cw ? (int32_t)k.rows : 0, k.nseg > 1 ? k.nseg : 0,
         {(const uint8_t*)k.wseg[0], (const uint8_t*)k.wseg[1], (const uint8_t*)k.wseg[2]},
         {(const float*)k.bseg[0], (const float*)k.bseg[1], (const float*)k.bseg[2]},
         {(float*)k.yseg[0], (float*)k.yseg[1], (float*)k.yseg[2]},
         {(int32_t)k.oseg[0], (int32_t)k.oseg[1], (int32_t)k.oseg[2]},
         k.dtype2 ? k.nseg1 : k.nseg, (const float*)k.rl, (float*)k.rw, (int32_t)k.rexp,
         (int32_t)k.rk, (int32_t)k.rnorm, 0, (const float*)k.rscale, (uint8_t*)k.xq_out, k.xq_k8, 0,
         {0, 0, 0, 0}};
  if (k.rl && (!k.ids || !k.rw || !k.w2 || !(k.nw || xq) || k.batch_rows() || k.rexp < 1 || k.rexp > 256 || k.rk < 1 ||
               k.rk > std::min<int64_t>(k.rexp, 8) || k.rk != k.rows))
    return fail(IHIP_E_ARG, "EnqueueLinear: self-routing takes one token's <= 8 slots of <= 256 experts, gate/up with a norm or a quantized row");
  if (k.w2 && batch) return fail(IHIP_E_ARG, "EnqueueLinear: the fused SwiGLU takes one row per block");
  // a chunk of rows in the Q8 arithmetic: the MFMA GEMM (64 x 64 tiles)
  // (float weights in the Q8 arithmetic: the float activations as they are,
  // on the f64 matrix cores)
  const bool gemm_q8 = (q8 || float_fmt(k.dtype)) && gemm_runs(c, k.dtype, mode);
  if (k.items && k.item_rows > 8 && !gemm_q8)
    return fail(IHIP_E_ARG, "EnqueueLinear: items of more than 8 slots need the GEMM");
  const int min_rows = float_fmt(k.dtype) ? c->gemm_min_rows_float : c->gemm_min_rows;
  if (batch && gemm_q8 && (k.items ? k.item_rows > 8 : k.rows >= min_rows)) {
    struct {
      const uint8_t* w;
      const uint8_t* xq;
      const float* bias;
      float* y;
      int64_t stride;
      int32_t out, in, rows, pad;
      const void* items;
      const int* perm;
      int32_t x_per_slot, pad2;
      const float* x;
      double* part;
      int32_t ksplit, klen;
    } g = {(const uint8_t*)k.w, (const uint8_t*)xq, (const float*)k.bias, (float*)k.y, k.stride,
           (int32_t)k.out, (int32_t)k.in, (int32_t)k.rows, 0, (const void*)k.items,
           (const int*)k.perm, k.x_per_slot, 0, (const float*)k.x, nullptr, 1, 0};
    if (k.items && k.item_rows > 64) return fail(IHIP_E_ARG, "EnqueueLinear: items of at most 64 slots");
    char gname[32];
    snprintf(gname, sizeof gname, "gemm_%s", fmt_name(k.dtype));
    const unsigned gx = (unsigned)((k.out + 63) / 64);
    const unsigned gy = (unsigned)(k.items ? k.nitems : (k.rows + 63) / 64);
    // float weights with too few tiles to fill the chip (a router: 128
    // outputs): the sum split into ksplit parts of >= 256 values, one block
    // each, then their double sums added in split order
    int ksplit = 1;
    if (float_fmt(k.dtype) && !k.items && !k.no_alloc && !c->capturing && c->gemm_split) {
      const int64_t tiles = (int64_t)gx * gy;
      while (ksplit < 16 && tiles * ksplit * 2 <= (int64_t)c->cus * 2 && k.in / (ksplit * 2) >= 256)
        ksplit *= 2;
    }
    if (ksplit > 1) {
      const int64_t n = k.rows * k.out;
      int rc = scratch(c, c->scratch_split, c->scratch_split_bytes, (uint64_t)n * ksplit * 8);
      if (rc) return rc;
      g.part = (double*)c->scratch_split;
      g.ksplit = ksplit;
      g.klen = (int32_t)(((k.in + ksplit - 1) / ksplit + 31) / 32 * 32);
      if ((rc = launch(c, gname, dim3(gx, gy, (unsigned)ksplit), dim3(256), &g))) return rc;
      struct {
        const double* part;
        const float* bias;
        float* y;
        int64_t n;
        int32_t out, ksplit;
      } sa = {(const double*)c->scratch_split, (const float*)k.bias, (float*)k.y, n,
              (int32_t)k.out, ksplit};
      return launch(c, "gemm_split_sum", dim3((unsigned)((n + 255) / 256)), dim3(256), &sa);
    }
    if (k.dtype == DT_MXFP4 && q8 && c->gemm_f8 && !k.no_alloc && !c->capturing) {
      // the e4m3 planes of the quantized rows, then the f8f6f4 GEMM on them
      const int64_t G = k.in / 32;
      const int64_t nx = k.items ? (k.x_per_slot ? (k.rows + k.x_per_slot - 1) / k.x_per_slot : 1) : k.rows;
      int rc = scratch(c, c->scratch_planes, c->scratch_planes_bytes, (uint64_t)nx * 68 * G);
      if (rc) return rc;
      struct {
        const uint8_t* xq;
        uint8_t* planes;
        int32_t rows, in;
      } pa = {(const uint8_t*)xq, (uint8_t*)c->scratch_planes, (int32_t)nx, (int32_t)k.in};
      if ((rc = launch(c, "f8_planes", dim3((unsigned)((G + 255) / 256), (unsigned)nx), dim3(256), &pa)))
        return rc;
      g.xq = (const uint8_t*)c->scratch_planes;
      return launch(c, "gemm_mxfp4_f8", dim3(gx, gy), dim3(256), &g);
    }
    return launch(c, gname, dim3(gx, gy), dim3(256), &g);
  }
  if (k.nw && (batch || k.in > 4096 || xq))
    return fail(IHIP_E_ARG, "EnqueueLinear: the fused rmsnorm takes one float row of at most 4096");
  if ((k.res || k.cw) && (batch || k.w2 || (k.ids && !k.cw)))
    return fail(IHIP_E_ARG, "EnqueueLinear: a residual add takes one plain or combined row");
  if (k.nseg > 1 && (k.nseg > 3 || batch || k.ids || k.w2 || k.res || k.cw))
    return fail(IHIP_E_ARG, "EnqueueLinear: 2..3 matrices take one plain row");
  char name[64];
  const int64_t rpw = 64 / lpr, tiles = (k.out + rpw - 1) / rpw;
  if (k.cw) {
    // the experts of one token added into the residual: one block per tile
    const int64_t xbytes = q8 ? k.rows * k.in + k.rows * k.in / 8 : k.rows * k.in * 4;
    if (!k.ids || k.rows < 1 || k.rows > 8 || xq || k.w2 || k.x_per_slot != 1 || xbytes > 65536)
      return fail(IHIP_E_ARG, "EnqueueLinear: combine takes 1..8 slots of float rows (64 KB)");
    snprintf(name, sizeof name, "gemv_%s_%s_cmb_u%d", fmt_name(k.dtype),
             mode == IHIP_MODE_Q8 ? "q8" : "f32", U);
    const int64_t hold = (int64_t)c->cus * resident_blocks(c, name, 256, (size_t)xbytes);
    return launch(c, name, dim3((unsigned)std::max<int64_t>(1, std::min(tiles, hold))), dim3(256), &a,
                  (size_t)xbytes);
  }
  if (float_fmt(k.dtype) && mode == IHIP_MODE_Q8 && !batch && !k.ids && !k.w2 && !k.dtype2) {
    // float weights, one row: a wave reads each row as consecutive 16-byte
    // chunks (gemv_flt), one row per wave step
    const int64_t chunks = k.in * (k.dtype == DT_F32 ? 4 : 2) / 16;
    if (chunks <= 1024) {
      snprintf(name, sizeof name, "gemv_%s_q8_%srows_j%d", fmt_name(k.dtype), k.nw ? "norm_" : "",
               chunks <= 512 ? 8 : 16);
      // the rows of every matrix in one index space, a row per wave step:
      // one round of resident blocks, each staging the activation row once
      int64_t rows = k.out;
      if (k.nseg > 1) {
        rows = 0;
        for (int i = 0; i < k.nseg; i++) rows += k.oseg[i];
      }
      const int64_t hold = (int64_t)c->cus * resident_blocks(c, name, 256) * c->gemv_hold;
      const int64_t wgs = std::max<int64_t>(1, std::min((rows + 3) / 4, hold));
      if (k.xq_out && (!k.nw || (k.xq_k8 && k.in % 256)))
        return fail(IHIP_E_ARG, "EnqueueLinear: the quantized row out takes a normed row (Q8_K: whole super-blocks)");
      // (the quantized row out: one block more, which takes no rows)
      return launch(c, name, dim3((unsigned)(wgs + (k.xq_out ? 1 : 0))), dim3(256), &a);
    }
  }
  if (k.xq_out) return fail(IHIP_E_ARG, "EnqueueLinear: the quantized row out takes a normed one-row float GEMV");
  // a small batch of quantized rows on the int8 matrix cores: 8 rows (or an
  // item of at most 8 slots) x 128 outputs per block, the weights read once
  // per 8 rows (gemm8), when its tiles fill the chip (a block walks the
  // groups of its tiles in turn: a short matrix is left to gemv_rows below,
  // whose waves split the rows' groups)
  const int64_t blocks8 = ((k.out + 127) / 128) * (k.items ? k.nitems : (k.rows + 7) / 8);
  if (batch && q8 && !k.w2 && !k.dtype2 && !float_fmt(k.dtype) && c->use_gemm8 && gemm_fmt(k.dtype) &&
      blocks8 >= c->cus) {
    struct {
      const uint8_t* w;
      const uint8_t* xq;
      const float* bias;
      float* y;
      int64_t stride;
      int32_t out, in, rows, pad;
      const void* items;
      const int* perm;
      int32_t x_per_slot, pad2;
      const float* x;
      double* part;
      int32_t ksplit, klen;
    } g = {(const uint8_t*)k.w, (const uint8_t*)xq, (const float*)k.bias, (float*)k.y, k.stride,
           (int32_t)k.out, (int32_t)k.in, (int32_t)k.rows, 0, (const void*)k.items,
           (const int*)k.perm, k.x_per_slot, 0, (const float*)k.x, nullptr, 1, 0};
    snprintf(name, sizeof name, "gemm8_%s", fmt_name(k.dtype));
    const int64_t tiles8 = (k.out + 127) / 128;
    const unsigned gy8 = (unsigned)(k.items ? k.nitems : (k.rows + 7) / 8);
    const int64_t hold = (int64_t)c->cus * std::max(1, resident_blocks(c, name, 256));
    const int64_t per_chunk = (hold + gy8 - 1) / gy8;
    const int64_t gx8 = std::max<int64_t>(1, std::min(tiles8, per_chunk));
    return launch(c, name, dim3((unsigned)gx8, gy8), dim3(256), &g);
  }
  if (batch && q8 && !k.w2 && !k.dtype2 && k.in <= 8192 && !float_fmt(k.dtype)) {
    // a small batch of quantized rows: the rows staged in LDS once per block,
    // each weight group loaded and decoded once for all of them (gemv_rows)
    snprintf(name, sizeof name, "gemv_%s_q8_r8u%d", fmt_name(k.dtype), U);
    const int64_t rpw_r = 64 / a.lpr, tiles_r = (k.out + rpw_r - 1) / rpw_r;
    const int TB = U == 1 ? 2 : 1;
    const size_t shmem = (size_t)8 * (size_t)rows_stride((int)k.in);
    const unsigned gyr = (unsigned)(k.items ? k.nitems : (k.rows + 7) / 8);
    const int64_t hold = (int64_t)c->cus * std::max(1, resident_blocks(c, name, 256, shmem));
    const int64_t per_chunk = (hold + gyr - 1) / gyr;
    const int64_t wgs_r = std::max<int64_t>(1, std::min((tiles_r + 4 * TB - 1) / (4 * TB), per_chunk));
    return launch(c, name, dim3((unsigned)wgs_r, gyr), dim3(256), &a, shmem);
  }
  if (k.dtype2) {
    if (!k.nw || k.nseg < 2 || k.nseg1 < 1 || k.nseg1 >= k.nseg || !linear_ok(k.dtype2, k.in))
      return fail(IHIP_E_ARG, "EnqueueLinear: two types take normed matrices of both");
    snprintf(name, sizeof name, "gemv_%s_%s_%s_norm_u%d", fmt_name(k.dtype), fmt_name(k.dtype2),
             mode == IHIP_MODE_Q8 ? "q8" : "f32", U);
  } else {
    snprintf(name, sizeof name, "gemv_%s_%s_%s%su%d", fmt_name(k.dtype),
             mode == IHIP_MODE_Q8 ? "q8" : "f32", k.nw ? "norm_" : "",
             batch ? "b8" : (k.w2 ? "glu_" : ""), U);
  }
  // a self-routed token: one row more (row 0), whose first block forms the route
  unsigned gy = (unsigned)(k.items ? k.nitems : (k.ids ? k.rows + (k.rl ? 1 : 0) : (batch ? (k.rows + 7) / 8 : 1)));
  int64_t tiles_all = tiles;
  if (k.nseg > 1) {
    gy = (unsigned)k.nseg;
    tiles_all = 0;
    for (int i = 0; i < k.nseg; i++) {
      if (k.oseg[i] < 1 || !k.wseg[i] || !k.yseg[i]) return fail(IHIP_E_ARG, "EnqueueLinear: matrix");
      tiles_all = std::max<int64_t>(tiles_all, (k.oseg[i] + rpw - 1) / rpw);
    }
  }
  int64_t wgs = std::min<int64_t>((tiles_all + 3) / 4, (int64_t)c->cus * 8);
  if (!batch) {
    // one-row blocks stage the activation row once per block: give each wave
    // the T tiles of a step (the kernel's T), as long as the launch keeps
    // about two blocks per CU. Matrices of one launch (nseg) are sized by
    // the largest; the blocks of a smaller one past its rows end at once.
    const int T = k.w2 ? (U == 1 ? 2 : 1) : (U == 1 ? 4 : (U == 2 ? 2 : 1));
    // (the route row of a self-routed token is not a share: one block works)
    const unsigned share = k.nseg > 1 ? 1u : gy - (k.ids && k.rl ? 1u : 0u);
    const int64_t want = ((int64_t)c->cus * c->gemv_blocks_per_cu + share - 1) / share;
    wgs = std::min(wgs, std::max<int64_t>((tiles_all + 4 * T - 1) / (4 * T), want));
    // and no more blocks than the chip holds at once: the waves walk the
    // rest of the rows, each block stages its row once
    const int64_t hold = ((int64_t)c->cus * resident_blocks(c, name, 256) * c->gemv_hold + share - 1) / share;
    wgs = std::max<int64_t>(1, std::min(wgs, hold));
    static const bool seg1d = [] {
      const char* v = getenv("IHIP_GEMV_SEG1D");
      return !v || atoi(v) != 0;
    }();
    if (k.nseg > 1 && seg1d) {
      // one index space: each matrix its own blocks, sized as above for its
      // own rows, none idle
      int64_t start = 0;
      for (int i = 0; i < k.nseg; i++) {
        const int64_t ti = (k.oseg[i] + rpw - 1) / rpw;
        const int64_t bi = std::max<int64_t>(1, std::min(wgs, (ti + 4 * T - 1) / (4 * T)));
        a.bstart[i] = (int32_t)start;
        start += bi;
      }
      a.bstart[k.nseg] = (int32_t)start;
      if (k.nseg == 2) a.bstart[3] = (int32_t)start;
      return launch(c, name, dim3((unsigned)start, 1), dim3(256), &a);
    }
  }
  return launch(c, name, dim3((unsigned)wgs, gy), dim3(256), &a);
}

static WeightEntry* find_weight(ihip_ctx* c, const void* host, int t, uint64_t bytes, int64_t stride_rows = 0)
{
  for (auto& w : c->weights)
    if (w.host == host && w.dtype == t && w.bytes == bytes && w.stride_rows == stride_rows) return &w;
  return nullptr;
}

int weight_rows(ihip_ctx* c, const void* host, int t, int64_t out, int64_t in, int64_t count,
                int64_t stride_rows, uint64_t* dev)
{
  if (!c || !host || !dev || out < 1 || in < 1 || count < 1 || stride_rows < out || !block_values(t) ||
      in % block_values(t))
    return fail(IHIP_E_ARG, "weight_rows: bad shape or type");
  const uint64_t rb = row_bytes(t, in), bytes = rb * (uint64_t)out * (uint64_t)count;
  if (WeightEntry* w = find_weight(c, host, t, bytes, stride_rows)) {
    *dev = w->dev;
    return 0;
  }
  if (c->capturing) return fail(IHIP_E_CAPTURE, "weight_rows: upload while capturing");
  std::vector<uint8_t> rows(bytes), staged(bytes);
  for (int64_t e = 0; e < count; e++)
    memcpy(rows.data() + (uint64_t)e * out * rb, (const uint8_t*)host + (uint64_t)e * stride_rows * rb,
           (size_t)(out * rb));
  void* p = nullptr;
  IHIP_CHECK(hipSetDevice(c->device));
  IHIP_CHECK(hipMalloc(&p, (bytes + 255) & ~(uint64_t)255));
  repack(rows.data(), staged.data(), t, out, in, count);
  hipError_t e = hipMemcpyHtoD((hipDeviceptr_t)p, staged.data(), bytes);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "weight_rows upload");
  }
  WeightEntry w{host, t, bytes, (uint64_t)p};
  w.stride_rows = stride_rows;
  c->weights.push_back(w);
  *dev = (uint64_t)p;
  return 0;
}

}  // namespace ihip

using namespace ihip;

extern "C" {

uint64_t ihip_type_bytes(int t, uint64_t count)
{
  int bv = block_values(t);
  if (!bv || count % bv) return 0;
  return count / bv * block_bytes(t);
}

int ihip_gpu_linear(int t, int64_t in) { return linear_ok(t, in) ? 1 : 0; }

int ihip_repack(const void* src, void* dst, int t, int64_t out, int64_t in, int64_t count,
                int inverse)
{
  if (!src || !dst || out < 1 || in < 1 || count < 1 || !block_values(t) || in % block_values(t) ||
      (t != DT_F32 && t != DT_F16 && t != DT_BF16 && in % 32))
    return fail(IHIP_E_ARG, "ihip_repack: bad shape or type");
  if (inverse) unpack(src, dst, t, out, in, count);
  else repack(src, dst, t, out, in, count);
  return 0;
}

int ihip_weight(ihip_ctx* c, const void* host, int t, int64_t out, int64_t in, int64_t count,
                uint64_t* dev)
{
  if (!c || !host || !dev || out < 1 || in < 1 || count < 1 || !block_values(t) ||
      in % block_values(t))
    return fail(IHIP_E_ARG, "ihip_weight: bad shape or type");
  const uint64_t bytes = row_bytes(t, in) * (uint64_t)out * (uint64_t)count;
  if (WeightEntry* w = find_weight(c, host, t, bytes)) {
    *dev = w->dev;
    return 0;
  }
  if (c->capturing) return fail(IHIP_E_CAPTURE, "ihip_weight: upload while capturing");
  void* p = nullptr;
  IHIP_CHECK(hipSetDevice(c->device));
  // rounded up to 256 bytes: a 16-byte load never reaches past the buffer
  IHIP_CHECK(hipMalloc(&p, (bytes + 255) & ~(uint64_t)255));
  std::vector<uint8_t> staged(bytes);
  repack(host, staged.data(), t, out, in, count);
  hipError_t e = hipMemcpyHtoD((hipDeviceptr_t)p, staged.data(), bytes);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "ihip_weight upload");
  }
  c->weights.push_back({host, t, bytes, (uint64_t)p});
  *dev = (uint64_t)p;
  return 0;
}

int ihip_weight_f32(ihip_ctx* c, const float* host, int64_t count, uint64_t* dev)
{
  return ihip_weight(c, host, DT_F32, 1, count, 1, dev);
}

int ihip_forget_weights(ihip_ctx* c, const void* from, const void* to)
{
  if (!c) return fail(IHIP_E_ARG, "ihip_forget_weights");
  if ((uintptr_t)to <= (uintptr_t)from) return c->weight_epoch;
  size_t n = 0, before = c->weights.size();
  for (size_t i = 0; i < c->weights.size(); i++) {
    WeightEntry& w = c->weights[i];
    if ((uintptr_t)w.host < (uintptr_t)to && (uintptr_t)w.host + w.bytes > (uintptr_t)from) {
      (void)hipStreamSynchronize(c->stream);
      (void)hipFree((void*)w.dev);
    } else {
      c->weights[n++] = w;
    }
  }
  c->weights.resize(n);
  if (n != before) c->weight_epoch++;
  return c->weight_epoch;
}

int ihip_clear_weights(ihip_ctx* c)
{
  if (!c) return fail(IHIP_E_ARG, "ihip_clear_weights");
  (void)hipStreamSynchronize(c->stream);
  for (auto& w : c->weights) (void)hipFree((void*)w.dev);
  c->weights.clear();
  return ++c->weight_epoch;
}

int ihip_enqueue_linear_at(ihip_ctx* c, uint64_t x, int64_t rows, int64_t in, int t, uint64_t w,
                           int64_t out, uint64_t y, uint64_t bias, int mode)
{
  if (!c) return fail(IHIP_E_ARG, "no context");
  LinearCall k;
  k.x = x; k.rows = rows; k.in = in; k.dtype = t; k.w = w; k.out = out; k.y = y;
  k.bias = bias; k.mode = mode;
  return enqueue_linear(c, k);
}

int ihip_enqueue_linear_ids(ihip_ctx* c, uint64_t x, int64_t in, int t, uint64_t w,
                            int64_t stride, int64_t out, uint64_t ids, int64_t slots,
                            int x_per_slot, uint64_t y, uint64_t bias, int mode)
{
  if (!c || !ids || stride <= 0) return fail(IHIP_E_ARG, "EnqueueLinearIds: no ids or stride");
  LinearCall k;
  k.x = x; k.rows = slots; k.in = in; k.dtype = t; k.w = w; k.out = out; k.y = y;
  k.bias = bias; k.mode = mode; k.ids = ids; k.stride = stride; k.x_per_slot = x_per_slot;
  return enqueue_linear(c, k);
}

int ihip_linear(ihip_ctx* c, const float* x, int64_t rows, int64_t in, const void* w, int t,
                int64_t out, const float* bias, float* y, int mode)
{
  if (!c || !x || !w || !y) return fail(IHIP_E_ARG, "ihip_linear: null buffer");
  if (!linear_ok(t, in)) return fail(IHIP_E_UNSUPPORTED, "ihip_linear: not supported");
  std::lock_guard<std::mutex> g(c->lock);
  uint64_t dw = 0, db = 0;
  int rc = ihip_weight(c, w, t, out, in, 1, &dw);
  if (!rc && bias) rc = ihip_weight_f32(c, bias, out, &db);
  if (!rc) rc = scratch(c, c->scratch_x, c->scratch_x_bytes, (uint64_t)rows * in * 4);
  if (!rc) rc = scratch(c, c->scratch_y, c->scratch_y_bytes, (uint64_t)rows * out * 4);
  if (rc) return rc;
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)c->scratch_x, (void*)x, (size_t)rows * in * 4, c->stream));
  rc = ihip_enqueue_linear_at(c, c->scratch_x, rows, in, t, dw, out, c->scratch_y, db, mode);
  if (rc) return rc;
  IHIP_CHECK(hipMemcpyDtoHAsync(y, (hipDeviceptr_t)c->scratch_y, (size_t)rows * out * 4, c->stream));
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  return 0;
}

int ihip_enqueue_dequant(ihip_ctx* c, uint64_t w, int t, int64_t out, int64_t in, int64_t row0,
                         int64_t rows, uint64_t y)
{
  if (!c || !fmt_name(t) || in % 32 || ((t == DT_Q4_K || t == DT_Q6_K) && in % 256) || rows < 1 ||
      row0 < 0 || row0 + rows > out)
    return fail(IHIP_E_ARG, "ihip_enqueue_dequant: bad shape");
  struct {
    const uint8_t* w;
    const int* ids;
    float* y;
    int64_t row0;
    int32_t out, in, rows, pad;
  } a = {(const uint8_t*)w, nullptr, (float*)y, row0, (int32_t)out, (int32_t)in, (int32_t)rows, 0};
  char name[48];
  snprintf(name, sizeof name, "dequant_%s", fmt_name(t));
  return launch(c, name, dim3((unsigned)((rows + 3) / 4)), dim3(256), &a);
}

int ihip_enqueue_embed(ihip_ctx* c, uint64_t embed, int t, int64_t vocab, int64_t hidden,
                       uint64_t ids, int64_t rows, uint64_t x)
{
  if (!c || !fmt_name(t) || hidden % 32 || rows < 1 || !ids)
    return fail(IHIP_E_ARG, "ihip_enqueue_embed: bad shape");
  struct {
    const uint8_t* w;
    const int* ids;
    float* y;
    int64_t row0;
    int32_t out, in, rows, pad;
  } a = {(const uint8_t*)embed, (const int*)ids, (float*)x, 0, (int32_t)vocab, (int32_t)hidden,
         (int32_t)rows, 0};
  char name[48];
  snprintf(name, sizeof name, "dequant_%s", fmt_name(t));
  return launch(c, name, dim3((unsigned)((rows + 3) / 4)), dim3(256), &a);
}

uint64_t ihip_q8_bytes(int64_t in, int k_quant)
{
  (void)k_quant;
  return q8_row_bytes(in);
}

int ihip_enqueue_quantize(ihip_ctx* c, uint64_t x, int64_t rows, int64_t in, int k_quant,
                          uint64_t xq, uint64_t bad)
{
  if (!c || in % (k_quant ? 256 : 32) || rows < 1) return fail(IHIP_E_ARG, "ihip_enqueue_quantize");
  uint64_t keep = c->scratch_bad;
  if (bad) c->scratch_bad = bad;
  int rc = enqueue_quantize(c, x, rows, in, k_quant ? 1 : 0, xq);
  c->scratch_bad = keep;
  return rc;
}

struct NormArgs {
  float* x;
  const float* t;
  const float* w;
  float* y;
  double eps;
  int32_t rows, cols;
  const float* cd;
  const float* cw;
  int32_t k, pad;
};

int ihip_enqueue_rmsnorm(ihip_ctx* c, uint64_t x, uint64_t w, uint64_t y, int64_t rows,
                         int64_t cols, double eps)
{
  if (!c || rows < 1 || cols < 1) return fail(IHIP_E_ARG, "ihip_enqueue_rmsnorm");
  NormArgs a = {(float*)x, nullptr, (const float*)w, (float*)y, eps, (int32_t)rows, (int32_t)cols,
                nullptr, nullptr, 0, 0};
  return launch(c, "rmsnorm", dim3((unsigned)rows), dim3(1024), &a);
}

int ihip_enqueue_addnorm(ihip_ctx* c, uint64_t x, uint64_t t, uint64_t w, uint64_t y, int64_t rows,
                         int64_t cols, double eps)
{
  if (!c || rows < 1 || cols < 1 || !t) return fail(IHIP_E_ARG, "ihip_enqueue_addnorm");
  NormArgs a = {(float*)x, (const float*)t, (const float*)w, (float*)y, eps, (int32_t)rows,
                (int32_t)cols, nullptr, nullptr, 0, 0};
  return launch(c, "rmsnorm", dim3((unsigned)rows), dim3(1024), &a);
}

struct EltArgs {
  float* x;
  const float* t;
  int64_t n;
  float alpha, limit;
};

}  // extern "C"

namespace ihip {

int enqueue_addnorm_moe(ihip_ctx* c, uint64_t x, uint64_t cd, uint64_t cw, int64_t k, uint64_t w,
                        uint64_t y, int64_t rows, int64_t cols, double eps)
{
  NormArgs a = {(float*)x, nullptr, (const float*)w, (float*)y, eps, (int32_t)rows, (int32_t)cols,
                (const float*)cd, (const float*)cw, (int32_t)k, 0};
  return launch(c, "rmsnorm", dim3((unsigned)rows), dim3(1024), &a);
}

}  // namespace ihip

extern "C" {

int ihip_enqueue_add(ihip_ctx* c, uint64_t x, uint64_t t, int64_t n)
{
  if (!c || n < 1) return fail(IHIP_E_ARG, "ihip_enqueue_add");
  EltArgs a = {(float*)x, (const float*)t, n, 0.f, 0.f};
  return launch(c, "add", dim3((unsigned)((n + 255) / 256)), dim3(256), &a);
}

int ihip_enqueue_swiglu(ihip_ctx* c, uint64_t gate, uint64_t up, int64_t n, float alpha, float limit)
{
  if (!c || n < 1) return fail(IHIP_E_ARG, "ihip_enqueue_swiglu");
  EltArgs a = {(float*)gate, (const float*)up, n, alpha, limit};
  return launch(c, "swiglu", dim3((unsigned)((n + 255) / 256)), dim3(256), &a);
}

int ihip_enqueue_qkrope(ihip_ctx* c, uint64_t q, uint64_t k, uint64_t v, uint64_t qn, uint64_t kn,
                        uint64_t cs, uint64_t kc, uint64_t vc, int64_t rows, int64_t heads,
                        int64_t kvh, int64_t hd, int64_t past, double eps, int kv_f16)
{
  if (!c || rows < 1 || heads < 1 || kvh < 1 || hd < 2 || hd > 512 || (hd & 1) || past < 0)
    return fail(IHIP_E_ARG, "ihip_enqueue_qkrope");
  struct {
    float* q;
    const float* k;
    const float* v;
    const float* qn;
    const float* kn;
    const float* cs;
    void* kc;
    void* vc;
    const int* pastp;
    double eps;
    int32_t rows, heads, kvh, hd, past, f16, rot, pad;
  } a = {(float*)q, (const float*)k, (const float*)v, (const float*)qn, (const float*)kn,
         (const float*)cs, (void*)kc, (void*)vc, nullptr, eps, (int32_t)rows, (int32_t)heads,
         (int32_t)kvh, (int32_t)hd, (int32_t)past, kv_f16};
  return launch(c, "qkrope", dim3((unsigned)(heads + kvh), (unsigned)rows), dim3(64), &a);
}

int ihip_enqueue_attention(ihip_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t y,
                           int64_t rows, int64_t heads, int64_t kvh, int64_t hd, int64_t past,
                           int64_t window, uint64_t sinks, double scale, int kv_f16)
{
  if (!c || rows < 1 || heads < 1 || kvh < 1 || heads % kvh || hd < 2 || hd > 512 || past < 0 ||
      window < 0)
    return fail(IHIP_E_ARG, "ihip_enqueue_attention");
  if (hd & 1) return fail(IHIP_E_ARG, "attention: an odd head size");
  int64_t maxkeys = past + rows;
  if (window > 0 && maxkeys > window) maxkeys = window;
  const int splits = attention_splits(maxkeys);
  int rc = scratch(c, c->scratch_attn, c->scratch_attn_bytes,
                   (uint64_t)heads * rows * splits * (hd + 2) * 8);
  if (rc) return rc;
  return enqueue_attention(c, q, kc, vc, y, c->scratch_attn, rows, heads, kvh, hd, past, 0, window,
                           sinks, scale, kv_f16, splits);
}

int ihip_enqueue_route(ihip_ctx* c, uint64_t logits, int64_t experts, int64_t k, int norm_topk,
                       uint64_t ids, uint64_t w, uint64_t scale)
{
  if (!c || experts < 1 || experts > 4096 || k < 1 || k > 64 || k > experts)
    return fail(IHIP_E_ARG, "ihip_enqueue_route");
  struct {
    const float* logits;
    int* ids;
    float* w;
    int32_t experts, k, norm, rows;
    const float* scale;
  } a = {(const float*)logits, (int*)ids, (float*)w, (int32_t)experts, (int32_t)k, norm_topk, 1,
         (const float*)scale};
  return launch(c, "route", dim3(1), dim3(256), &a);
}

int ihip_enqueue_moecombine(ihip_ctx* c, uint64_t d, uint64_t w, uint64_t y, int64_t k, int64_t n)
{
  if (!c || k < 1 || n < 1) return fail(IHIP_E_ARG, "ihip_enqueue_moecombine");
  struct {
    const float* d;
    const float* w;
    float* y;
    int32_t k, n, rows, pad;
  } a = {(const float*)d, (const float*)w, (float*)y, (int32_t)k, (int32_t)n, 1, 0};
  return launch(c, "moecombine", dim3((unsigned)((n + 255) / 256), 1), dim3(256), &a);
}

int ihip_enqueue_argmax(ihip_ctx* c, uint64_t v, int64_t n, uint64_t out)
{
  if (!c || n < 1 || n >= 0xffffffffLL) return fail(IHIP_E_ARG, "ihip_enqueue_argmax");
  // blocks of at least 1024 values, at most ARGMAX_PARTS of them
  const int64_t chunk = std::max<int64_t>(1024, (n + ARGMAX_PARTS - 1) / ARGMAX_PARTS);
  const int parts = (int)((n + chunk - 1) / chunk);
  struct {
    const float* v;
    int* out;
    int64_t n;
    uint64_t* part;
    int64_t chunk;
    int32_t parts, pad;
  } a = {(const float*)v, (int*)out, n, (uint64_t*)c->scratch_argmax, chunk, parts, 0};
  int rc = launch(c, "argmax_part", dim3((unsigned)parts), dim3(256), &a);
  if (rc) return rc;
  return launch(c, "argmax_final", dim3(1), dim3(256), &a);
}

}  // extern "C"


namespace {
constexpr int SAMPLE_BUCKETS = 128, SAMPLE_MAX_BLOCKS = 256;
// tokens per block of sample_probs / sample_compact: a multiple of 256, at
// least 1024, at most SAMPLE_MAX_BLOCKS blocks
int64_t sample_per(int64_t n)
{
  int64_t per = std::max<int64_t>(1024, (n + SAMPLE_MAX_BLOCKS - 1) / SAMPLE_MAX_BLOCKS);
  return (per + 255) / 256 * 256;
}
}  // namespace

extern "C" {

int ihip_sampler_create(ihip_ctx* c, const ihip_sampling* s, int64_t n_max, ihip_sampler** out)
{
  // n_max up to 2^22: the 2^40 fixed-point masses of p <= 1 sum below 2^63
  if (!c || !s || !out || n_max < 1 || n_max > (1 << 22)) return fail(IHIP_E_ARG, "ihip_sampler_create");
  *out = nullptr;
  // TInferSampler.Create (sampler.pas:210-223): NaN, infinities and settings
  // out of range refused
  if (!std::isfinite(s->temperature) || !std::isfinite(s->top_p) || !std::isfinite(s->min_p) ||
      s->top_k < 0 || s->top_p <= 0 || s->top_p > 1 || s->min_p < 0 || s->min_p >= 1)
    return fail(IHIP_E_ARG, "ihip_sampler_create: temperature, top_k, top_p or min_p out of range");
  if (c->capturing) return fail(IHIP_E_CAPTURE, "ihip_sampler_create while capturing");
  auto* k = new ihip_sampler;
  k->c = c;
  k->temperature = s->temperature;
  k->top_p = s->top_p;
  k->min_p = s->min_p;
  k->top_k = s->top_k;
  k->n_max = n_max;
  const int64_t nb = (n_max + sample_per(n_max) - 1) / sample_per(n_max);
  hipError_t e = hipSetDevice(c->device);
  auto get = [&](uint64_t& dst, size_t bytes) {
    void* q = nullptr;
    if (e == hipSuccess) e = hipMalloc(&q, std::max<size_t>(bytes, 256));
    if (q) k->mem.push_back(q);
    dst = (uint64_t)q;
  };
  get(k->state, 8);
  get(k->p, (size_t)n_max * 8);
  get(k->bsum, (size_t)nb * 8);
  get(k->bq, (size_t)nb * 8);
  get(k->bcnt, (size_t)nb * SAMPLE_BUCKETS * 4);
  get(k->bmass, (size_t)nb * SAMPLE_BUCKETS * 8);
  get(k->cid, (size_t)n_max * 4);
  get(k->ckey, (size_t)n_max * 4);
  get(k->cp, (size_t)n_max * 8);
  const uint64_t seed = (uint64_t)s->seed;
  if (e == hipSuccess) e = hipMemcpy((void*)k->state, &seed, 8, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    ihip_sampler_destroy(k);
    return hip_fail(e, "ihip_sampler_create");
  }
  *out = k;
  return 0;
}

void ihip_sampler_destroy(ihip_sampler* k)
{
  if (!k) return;
  (void)hipStreamSynchronize(k->c->stream);
  for (void* q : k->mem) (void)hipFree(q);
  delete k;
}

int ihip_enqueue_sample(ihip_ctx* c, ihip_sampler* k, uint64_t logits, int64_t n, uint64_t out)
{
  if (!c || !k || k->c != c || !logits || !out || n < 1 || n > k->n_max)
    return fail(IHIP_E_ARG, "ihip_enqueue_sample");
  // the argmax first: greedy, or the best token of the draw
  int rc = ihip_enqueue_argmax(c, logits, n, out);
  if (rc || !(k->temperature > 0)) return rc;
  const int64_t per = sample_per(n), nb = (n + per - 1) / per;
  struct {
    const float* logits;
    const int* best;
    int* out;
    uint64_t* state;
    double* p;
    double* bsum;
    double* bq;
    uint32_t* bcnt;
    uint64_t* bmass;
    int* cid;
    uint32_t* ckey;
    double* cp;
    double temperature, top_p, min_p;
    int32_t n, top_k, nb, per;
  } a = {(const float*)logits, (const int*)out, (int*)out, (uint64_t*)k->state, (double*)k->p,
         (double*)k->bsum, (double*)k->bq, (uint32_t*)k->bcnt, (uint64_t*)k->bmass, (int*)k->cid,
         (uint32_t*)k->ckey, (double*)k->cp, k->temperature, k->top_p, k->min_p, (int32_t)n, k->top_k,
         (int32_t)nb, (int32_t)per};
  if ((rc = launch(c, "sample_probs", dim3((unsigned)nb), dim3(256), &a))) return rc;
  if ((rc = launch(c, "sample_compact", dim3((unsigned)nb), dim3(256), &a))) return rc;
  return launch(c, "sample_pick", dim3(1), dim3(1024), &a);
}

}  // extern "C"

extern "C" int ihip_enqueue_stream_read(ihip_ctx* c, uint64_t p, uint64_t bytes, uint64_t out)
{
  if (!c || !p || bytes < 16 || bytes % 16 || !out) return fail(IHIP_E_ARG, "ihip_enqueue_stream_read");
  struct {
    const void* p;
    uint64_t n16;
    uint32_t* out;
  } a = {(const void*)p, bytes / 16, (uint32_t*)out};
  // 32 blocks per CU: the most bytes in flight (measured best on gfx950)
  const uint64_t blocks = std::min<uint64_t>((uint64_t)c->cus * 32, (bytes / 16 + 255) / 256);
  return launch(c, "stream_read", dim3((unsigned)blocks), dim3(256), &a);
}

namespace ihip {

int attention_splits(int64_t maxkeys) { return (int)std::max<int64_t>(1, (maxkeys + 127) / 128); }

// the ranges attention_merge weighs in one block
static const int MAX_SPLITS = 256;

int enqueue_attention_one(ihip_ctx* c, const AttnOne& o)
{
  if (o.hd != 64 && o.hd != 128) return fail(IHIP_E_UNSUPPORTED, "attention_one: head_dim 64 or 128");
  if (o.splits < 1 || o.splits > MAX_SPLITS || o.heads < 1 || o.kvh < 1 || o.heads % o.kvh)
    return fail(IHIP_E_ARG, "attention_one: heads / splits");
  struct {
    const float *q, *k, *v, *qn, *kn, *cs;
    void *kc, *vc;
    float* y;
    const float* sinks;
    const int* pastp;
    double* part;
    double scale, eps;
    int32_t heads, kvh, hd, past, window, splits;
    int* done;
    int32_t place, pad;
  } a = {(const float*)o.q, (const float*)o.k, (const float*)o.v, (const float*)o.qn,
         (const float*)o.kn, (const float*)o.cs, (void*)o.kc, (void*)o.vc, (float*)o.y,
         (const float*)o.sinks, (const int*)o.pastp, (double*)o.part,
         o.scale > 0 ? o.scale : 1.0 / std::sqrt((double)o.hd), o.eps, (int32_t)o.heads,
         (int32_t)o.kvh, (int32_t)o.hd, (int32_t)o.past, (int32_t)o.window, o.splits,
         (int*)o.done, 1, 0};
  char name[32];
  snprintf(name, sizeof name, "attention_one_%s_%d", o.f16 ? "f16" : "f32", (int)o.hd);
  int rc;
  if (o.f16) {
    // one block per (head, range) in a 1-D grid laid out over the XCDs by KV
    // group (ops.hip attn_one_block): with 8 / kvh XCDs a group, the ranges
    // rounded up to a multiple of that (a range past the keys is empty)
    static const int place = [] {
      const char* v = getenv("IHIP_ATTN_PLACE");
      return v ? atoi(v) : 1;
    }();
    a.place = place;
    if (place == 1 && o.heads % 8 == 0 && o.kvh <= 8 && 8 % o.kvh == 0) {
      const int X = 8 / (int)o.kvh;
      a.splits = (o.splits + X - 1) / X * X;
      if (a.splits > MAX_SPLITS) return fail(IHIP_E_ARG, "attention_one: heads / splits");
    }
    rc = launch(c, name, dim3((unsigned)(o.heads * a.splits)), dim3(256), &a);
  } else {
    rc = launch(c, name, dim3((unsigned)o.heads, 1, (unsigned)o.splits), dim3(256), &a);
  }
  if (rc || o.done) return rc;
  struct {
    const float* q;
    const void* kc;
    const void* vc;
    float* y;
    const float* sinks;
    const int* pastp;
    double* part;
    double scale;
    int32_t rows, heads, kvh, hd, past, window, f16, splits;
  } mg = {nullptr, nullptr, nullptr, (float*)o.y, (const float*)o.sinks, nullptr, (double*)o.part,
          0.0, 1, (int32_t)o.heads, (int32_t)o.kvh, (int32_t)o.hd, 0, 0, o.f16, a.splits};
  return launch(c, "attention_merge", dim3((unsigned)o.heads, 1), dim3(128), &mg);
}

int enqueue_attention(ihip_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t y, uint64_t part,
                      int64_t rows, int64_t heads, int64_t kvh, int64_t hd, int64_t past,
                      uint64_t pastp, int64_t window, uint64_t sinks, double scale, int f16,
                      int splits)
{
  if (!(scale > 0)) scale = 1.0 / std::sqrt((double)hd);
  if (splits > MAX_SPLITS) return fail(IHIP_E_UNSUPPORTED, "attention: more than 32768 keys per row");
  struct {
    const float* q;
    const void* kc;
    const void* vc;
    float* y;
    const float* sinks;
    const int* pastp;
    double* part;
    double scale;
    int32_t rows, heads, kvh, hd, past, window, f16, splits;
  } a = {(const float*)q, (const void*)kc, (const void*)vc, (float*)y, (const float*)sinks,
         (const int*)pastp, (double*)part, scale, (int32_t)rows, (int32_t)heads, (int32_t)kvh,
         (int32_t)hd, (int32_t)past, (int32_t)window, f16, splits};
  int rc;
  if ((hd == 64 || hd == 128) && rows > 1 && c->attn_mfma) {
    // tiles of 16 rows on the f64 matrix cores
    char name[32];
    snprintf(name, sizeof name, "attention_mfma_%s_%d", f16 ? "f16" : "f32", (int)hd);
    rc = launch(c, name, dim3((unsigned)heads, (unsigned)((rows + 15) / 16), (unsigned)splits), dim3(256), &a);
  } else if ((hd == 64 || hd == 128) && rows > 1) {
    // tiles of 8 rows sharing each range's keys
    char name[32];
    snprintf(name, sizeof name, "attention_rows_%s_%d", f16 ? "f16" : "f32", (int)hd);
    rc = launch(c, name, dim3((unsigned)heads, (unsigned)((rows + 7) / 8), (unsigned)splits), dim3(256), &a);
  } else {
    const char* name = hd > 256 ? (f16 ? "attention_part_f16_512" : "attention_part_f32_512")
                                : (f16 ? "attention_part_f16" : "attention_part_f32");
    rc = launch(c, name, dim3((unsigned)heads, (unsigned)rows, (unsigned)splits), dim3(256), &a);
  }
  if (rc) return rc;
  return launch(c, "attention_merge", dim3((unsigned)heads, (unsigned)rows), dim3(128), &a);
}

}  // namespace ihip
