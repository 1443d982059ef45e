// model.cpp - TQwen3Cuda of the reference
// (src/infer/mormot.ai.infer.model.qwen3.cuda.pas:150-1761) for HIP: the
// whole decoder on the device behind TDecoderDevice (decoder.pas:907-928).
// Qwen3 dense, Qwen3-MoE and gpt-oss shapes: per-head q/k norms, biases,
// sinks, sliding windows, clamped SwiGLU, experts chosen on the device.
//
// A prompt runs in chunks of up to CHUNK rows (CHUNK_MAX of
// model.qwen3.cuda.pas:308 is 256; here 1024 by default, so that a prompt
// chunk's GEMMs fill the 256 CUs, ihip_model_chunk sets fewer); a decode step (one row) is one HIP graph,
// captured once and replayed: the position lives in device memory, the
// token id and the cos/sin of the position are copied in before each launch,
// and the argmax runs on the device, so one int32 comes back per token.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>

#include "internal.h"

namespace ihip {

static const int64_t CHUNK = 1024;

struct DevLayer {
  uint64_t input_norm = 0, post_norm = 0, q = 0, k = 0, v = 0, o = 0;
  uint64_t qb = 0, kb = 0, vb = 0, ob = 0, qn = 0, kn = 0, sinks = 0;
  uint64_t gate = 0, up = 0, down = 0, router = 0, router_b = 0;
  uint64_t eg = 0, eu = 0, ed = 0, egb = 0, eub = 0, edb = 0;
  int qd = 0, kd = 0, vd = 0, od = 0, gd = 0, ud = 0, dd = 0, rd = 0, egd = 0, eud = 0, edd = 0;
  int64_t eg_stride = 0, ed_stride = 0;
  uint64_t kc = 0, vc = 0;
  int window = 0, moe = 0;
};

}  // namespace ihip

struct ihip_model {
  ihip_ctx* c = nullptr;
  ihip_model_desc d{};
  std::vector<ihip_layer_desc> layer_desc;
  std::vector<ihip::DevLayer> L;
  int mode = IHIP_MODE_Q8, kv_f16 = 0;
  int64_t max_tokens = 0, length = 0;
  uint64_t embed = 0, final_norm = 0, head = 0;
  int embed_dt = 0, head_dt = 0;
  // activations for CHUNK rows
  uint64_t x = 0, h = 0, tmp = 0, q = 0, k = 0, v = 0, attn = 0, gate = 0, up = 0;
  uint64_t route = 0, ids = 0, rw = 0, eout = 0, cs = 0, tok = 0, logits = 0, next = 0, pos = 0;
  uint64_t xq0 = 0, xqk = 0, xqf = 0;  // quantized h (Q8_0, Q8_K) and FFN input
  uint64_t perm = 0, items = 0;         // the experts of a prompt chunk (moe_plan)
  uint64_t attn_part = 0;               // flash-decoding partials
  // zeroed counters of the decode attention's heads (the last range block of
  // a head merges the head)
  uint64_t done = 0;
  uint64_t logits_all = 0;
  int64_t logits_all_rows = 0;
  std::vector<uint64_t> owned;
  // the host ranges of the uploaded weights: forgotten when the model goes,
  // as a model does in its destructor (backend.pas:151-158) - new host
  // tensors at a reused address must not meet the stale device copy
  std::vector<std::pair<const uint8_t*, uint64_t>> uploaded;
  bool graph_ready = false;
  ihip_sampler* sampler = nullptr;  // null: the argmax
  bool use_graphs = true;  // TQwen3Cuda.UseGraphs (model.qwen3.cuda.pas:253-262)
  int64_t chunk_rows = ihip::CHUNK;  // prompt rows per chunk (ihip_model_chunk), at most CHUNK
  int item_rows = 8;  // slots per grouped-expert work item: 64 when the experts run on the GEMM
  double prefill_ms = 0, decode_ms = 0;
};

namespace ihip {

// decoder.pas:1735-1741 and 1759-1829: inverse frequencies, every step
// rounded to single as the reference's float32 tensors; YaRN when factor > 0
static void inv_freq(const ihip_model_desc& d, std::vector<float>& f, float& scale)
{
  const int64_t dim = d.head_dim, half = dim / 2;
  const double lt = std::log(d.rope_theta);
  f.assign(half, 0.f);
  for (int64_t i = 0; i < half; i++) {
    float e = (float)((double)(2 * i) / (double)dim);
    float p = (float)std::exp(lt * (double)e);
    f[i] = 1.0f / p;
  }
  scale = 1.0f;
  if (d.rope_factor == 0) return;
  const double pi2 = 2 * M_PI;
  auto corr = [&](double rot) {
    return ((double)dim * std::log((double)d.rope_original / (rot * pi2))) / (2 * lt);
  };
  double lo = corr(d.rope_beta_fast), hi = corr(d.rope_beta_slow);
  if (d.rope_truncate) {
    lo = std::floor(lo);
    hi = std::ceil(hi);
  }
  if (lo < 0) lo = 0;
  if (hi > dim - 1) hi = (double)(dim - 1);
  if (lo == hi) hi = hi + 0.001;
  const float loS = (float)lo, spanS = (float)(hi - lo), fct = (float)d.rope_factor;
  for (int64_t i = 0; i < half; i++) {
    float e = (float)((double)(2 * i) / (double)dim);
    float pos = (float)std::exp(lt * (double)e);
    pos = fct * pos;
    float inter = 1.0f / pos, extra = f[i];
    float ramp = ((float)i - loS) / spanS;
    ramp = ramp < 0 ? 0.f : (ramp > 1 ? 1.f : ramp);
    float keep = 1.0f - ramp;
    ramp = 1.0f - keep;
    inter = inter * ramp;
    extra = extra * keep;
    f[i] = inter + extra;
  }
  if (d.rope_attention > 0) scale = (float)d.rope_attention;
  else if (fct <= 1) scale = 1.0f;
  else scale = (float)(0.1 * std::log((double)fct) + 1.0);
}

// TDecoderModel.Rotary (decoder.pas:2539-2561): the angle in single, cos and
// sin rounded to single, then times the YaRN scale in single
static void rotary(const ihip_model_desc& d, int64_t first, int64_t rows, float* cs)
{
  std::vector<float> f;
  float rs;
  inv_freq(d, f, rs);
  const int64_t half = d.head_dim / 2;
  float* sn = cs + rows * half;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < half; i++) {
      float angle = f[i] * (float)(first + r);
      float c = (float)std::cos((double)angle), s = (float)std::sin((double)angle);
      if (rs != 1.0f) {
        c = c * rs;
        s = s * rs;
      }
      cs[r * half + i] = c;
      sn[r * half + i] = s;
    }
}

static int dalloc(ihip_model* m, uint64_t bytes, uint64_t& p)
{
  void* q = nullptr;
  IHIP_CHECK(hipMalloc(&q, bytes ? (bytes + 255) & ~(uint64_t)255 : 256));
  m->owned.push_back((uint64_t)q);
  p = (uint64_t)q;
  return 0;
}

static int upw(ihip_model* m, const ihip_tensor& t, int64_t out, int64_t in, int64_t count,
               uint64_t& dev, int& dt)
{
  dev = 0;
  dt = t.dtype;
  if (!t.data) return 0;
  m->uploaded.emplace_back((const uint8_t*)t.data, row_bytes(t.dtype, in) * out * count);
  return ihip_weight(m->c, t.data, t.dtype, out, in, count, &dev);
}

static int upf(ihip_model* m, const ihip_tensor& t, int64_t n, uint64_t& dev)
{
  dev = 0;
  if (!t.data) return 0;
  if (t.dtype != DT_F32) return fail(IHIP_E_ARG, "model: norms, biases and sinks are F32");
  m->uploaded.emplace_back((const uint8_t*)t.data, (uint64_t)n * 4);
  return ihip_weight_f32(m->c, (const float*)t.data, n, &dev);
}

// the quantized copy of an activation buffer for a weight type, made once
struct QCache {
  uint64_t buf0 = 0, bufk = 0;
  bool have0 = false, havek = false;
};

static int lin(ihip_model* m, uint64_t x, QCache* qc, int64_t rows, int64_t in, int dt,
               uint64_t w, int64_t out, uint64_t bias, uint64_t y)
{
  LinearCall k;
  k.x = x; k.rows = rows; k.in = in; k.dtype = dt; k.w = w; k.out = out; k.bias = bias;
  k.y = y; k.mode = m->mode;
  if (m->mode == IHIP_MODE_Q8 && qc && q8_kind(dt) >= 0) {
    int kind = q8_kind(dt);
    bool& have = kind ? qc->havek : qc->have0;
    uint64_t buf = kind ? qc->bufk : qc->buf0;
    if (!have) {
      int rc = enqueue_quantize(m->c, x, rows, in, kind, buf);
      if (rc) return rc;
      have = true;
    }
    k.xq = buf;
  }
  return enqueue_linear(m->c, k);
}

static int lin_ids(ihip_model* m, uint64_t x, uint64_t xqbuf, int64_t xrows, int64_t in, int dt,
                   uint64_t w, int64_t stride, int64_t out, uint64_t ids, int64_t slots,
                   int x_div, uint64_t bias, uint64_t y, bool quantized)
{
  LinearCall k;
  k.x = x; k.rows = slots; k.in = in; k.dtype = dt; k.w = w; k.out = out; k.bias = bias;
  k.y = y; k.mode = m->mode; k.ids = ids; k.stride = stride; k.x_per_slot = x_div;
  k.nexp = m->d.experts;
  if (slots > m->d.experts_used) {
    // a prompt chunk: the slots grouped by expert (moe_plan), up to
    // item_rows rows per work item (8 for the 8-row GEMV, 64 for the GEMM),
    // so an expert's matrix is read once per that many of its tokens
    k.ids = 0;
    k.items = m->items;
    k.perm = m->perm;
    k.item_rows = m->item_rows;
    k.nitems = (slots + m->item_rows - 1) / m->item_rows + m->d.experts;
  }
  if (m->mode == IHIP_MODE_Q8 && q8_kind(dt) >= 0) {
    if (!quantized) {
      int rc = enqueue_quantize(m->c, x, xrows, in, q8_kind(dt), xqbuf);
      if (rc) return rc;
    }
    k.xq = xqbuf;
  }
  return enqueue_linear(m->c, k);
}

static int rope_attn(ihip_model* m, const DevLayer& L, int64_t n, int64_t past, bool graph)
{
  const ihip_model_desc& d = m->d;
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
    int32_t rows, heads, kvh, hd, past, f16;
  } ra = {(float*)m->q, (const float*)m->k, (const float*)m->v, (const float*)L.qn,
          (const float*)L.kn, (const float*)m->cs, (void*)L.kc, (void*)L.vc,
          graph ? (const int*)m->pos : nullptr, (double)d.rms_eps, (int32_t)n, d.heads,
          d.kv_heads, d.head_dim, (int32_t)past, m->kv_f16};
  int rc = launch(m->c, "qkrope", dim3((unsigned)(d.heads + d.kv_heads), (unsigned)n), dim3(64), &ra);
  if (rc) return rc;
  int64_t maxkeys = graph ? m->max_tokens : past + n;
  if (L.window > 0 && maxkeys > L.window) maxkeys = L.window;
  // a graph replays one grid for every position: splits for the longest
  return enqueue_attention(m->c, m->q, L.kc, L.vc, m->attn, m->attn_part, n, d.heads, d.kv_heads,
                           d.head_dim, past, graph ? m->pos : 0, L.window, L.sinks,
                           1.0 / std::sqrt((double)d.head_dim), m->kv_f16,
                           attention_splits(maxkeys));
}

// whether one row runs through layers_one: the norms fused into the GEMVs
// (hidden <= 4096), a token's experts combined in one launch (<= 8 slots)
static bool one_row_fused(const ihip_model* m)
{
  const ihip_model_desc& d = m->d;
  if (d.hidden > 4096) return false;
  if (d.experts > 0) {
    const int64_t K = d.experts_used;
    if (K < 1 || K > 8 || K * d.expert_ffn * 4 > 65536) return false;
  }
  return true;
}

// one row through the layers, x holding its embedding: every RMSNorm is
// computed by the GEMVs that read it (their staging), the residual adds by
// the GEMVs that produce them (o projection, FFN down, the experts'
// combine), so the row costs no norm or add launches. The arithmetic is that
// of layers() step for step. Leaves x = the residual (the final norm is the
// head's).
static int layers_one(ihip_model* m, int64_t past, bool graph)
{
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd,
                kvw = (int64_t)d.kv_heads * hd;
  int rc = 0;
  auto normed = [&](uint64_t nw, int dt, uint64_t w, int64_t out, uint64_t bias, uint64_t y) {
    LinearCall k;
    k.x = m->x; k.rows = 1; k.in = H; k.dtype = dt; k.w = w; k.out = out; k.bias = bias;
    k.y = y; k.mode = m->mode; k.nw = nw; k.eps = d.rms_eps;
    return enqueue_linear(m->c, k);
  };
  for (int l = 0; l < d.layers; l++) {
    const DevLayer& L = m->L[l];
    // attention block (decoder.pas:2625-2702)
    {
      // q, k and v: the matrices of one weight type in one launch
      const int dts[3] = {L.qd, L.kd, L.vd};
      const uint64_t ws[3] = {L.q, L.k, L.v}, bs[3] = {L.qb, L.kb, L.vb},
                     ys[3] = {m->q, m->k, m->v};
      const int64_t os[3] = {qw, kvw, kvw};
      bool done[3] = {false, false, false};
      // two types with a kernel for the pair (Q4_K_M: q, k Q4_K and v Q6_K)
      int t2 = 0;
      for (int j = 1; j < 3; j++)
        if (dts[j] != dts[0]) t2 = t2 ? (dts[j] == t2 ? t2 : -1) : dts[j];
      if (t2 > 0 && gemv_pair(m->c, dts[0], t2, m->mode, H)) {
        LinearCall k;
        k.x = m->x; k.rows = 1; k.in = H; k.dtype = dts[0]; k.dtype2 = t2; k.mode = m->mode;
        k.nw = L.input_norm; k.eps = d.rms_eps;
        for (int pass = 0; pass < 2; pass++)
          for (int j = 0; j < 3; j++)
            if ((dts[j] == dts[0]) == (pass == 0)) {
              k.wseg[k.nseg] = ws[j]; k.bseg[k.nseg] = bs[j]; k.yseg[k.nseg] = ys[j];
              k.oseg[k.nseg] = os[j]; k.nseg++;
              if (pass == 0) k.nseg1++;
              done[j] = true;
            }
        k.w = k.wseg[0]; k.y = k.yseg[0]; k.out = k.oseg[0];
        rc = enqueue_linear(m->c, k);
      }
      for (int i = 0; i < 3 && !rc; i++) {
        if (done[i]) continue;
        LinearCall k;
        k.x = m->x; k.rows = 1; k.in = H; k.dtype = dts[i]; k.mode = m->mode;
        k.nw = L.input_norm; k.eps = d.rms_eps;
        for (int j = i; j < 3; j++)
          if (!done[j] && dts[j] == dts[i]) {
            k.wseg[k.nseg] = ws[j]; k.bseg[k.nseg] = bs[j]; k.yseg[k.nseg] = ys[j];
            k.oseg[k.nseg] = os[j]; k.nseg++;
            done[j] = true;
          }
        if (k.nseg == 1) {
          k.w = k.wseg[0]; k.bias = k.bseg[0]; k.y = k.yseg[0]; k.out = k.oseg[0]; k.nseg = 0;
        } else {
          k.w = k.wseg[0]; k.y = k.yseg[0]; k.out = k.oseg[0];
        }
        rc = enqueue_linear(m->c, k);
      }
      if (rc) return rc;
    }
    if (hd == 64 || hd == 128) {
      // head norms, RoPE, cache store and the ranges in one launch, then the merge
      AttnOne o;
      o.q = m->q; o.k = m->k; o.v = m->v; o.qn = L.qn; o.kn = L.kn; o.cs = m->cs;
      o.kc = L.kc; o.vc = L.vc; o.y = m->attn; o.sinks = L.sinks; o.pastp = graph ? m->pos : 0;
      o.part = m->attn_part; o.scale = 1.0 / std::sqrt((double)hd);
      o.eps = d.rms_eps; o.heads = d.heads; o.kvh = d.kv_heads; o.hd = hd; o.past = past;
      o.window = L.window; o.f16 = m->kv_f16;
      if (d.heads <= 256) o.done = m->done;  // the merge in the last range block of a head
      int64_t maxkeys = graph ? m->max_tokens : past + 1;
      if (L.window > 0 && maxkeys > L.window) maxkeys = L.window;
      o.splits = attention_splits(maxkeys);
      if ((rc = enqueue_attention_one(m->c, o))) return rc;
    } else if ((rc = rope_attn(m, L, 1, past, graph))) {
      return rc;
    }
    {
      LinearCall k;
      k.x = m->attn; k.rows = 1; k.in = qw; k.dtype = L.od; k.w = L.o; k.out = H; k.bias = L.ob;
      k.y = m->x; k.res = m->x; k.mode = m->mode;
      if ((rc = enqueue_linear(m->c, k))) return rc;
    }
    if (!L.moe) {
      // DenseFfn (decoder.pas:2866-2878): gate, up and SwiGLU in one pass
      const int64_t F = d.ffn;
      if (L.gd != L.ud) return fail(IHIP_E_ARG, "model: gate and up of one type");
      LinearCall k;
      k.x = m->x; k.rows = 1; k.in = H; k.dtype = L.gd; k.w = L.gate; k.out = F;
      k.y = m->gate; k.mode = m->mode; k.w2 = L.up; k.alpha = d.swiglu_alpha;
      k.limit = d.swiglu_limit; k.nw = L.post_norm; k.eps = d.rms_eps;
      if ((rc = enqueue_linear(m->c, k))) return rc;
      LinearCall dn;
      dn.x = m->gate; dn.rows = 1; dn.in = F; dn.dtype = L.dd; dn.w = L.down; dn.out = H;
      dn.y = m->x; dn.res = m->x; dn.mode = m->mode;
      if ((rc = enqueue_linear(m->c, dn))) return rc;
      continue;
    }
    // MoeBlock (decoder.pas:3037-3053), the experts chosen on the device
    const int64_t E = d.experts, K = d.experts_used, FI = d.expert_ffn;
    if ((rc = normed(L.post_norm, L.rd, L.router, E, L.router_b, m->route))) return rc;
    // the route (TDecoderModel.Route) inside the gate/up launch: each block
    // ranks the logits for its slot's expert, one writes the picks and
    // weights for the down launch (up to 256 experts); else its own launch
    const bool self_route = E <= 256 && K <= E && K <= 8;
    if (!self_route) {
      struct {
        const float* logits;
        int* ids;
        float* w;
        int32_t experts, k, norm, rows;
      } ra = {(const float*)m->route, (int*)m->ids, (float*)m->rw, (int32_t)E, (int32_t)K,
              d.norm_topk, 1};
      if ((rc = launch(m->c, "route", dim3(1), dim3(256), &ra))) return rc;
    }
    LinearCall k;
    k.x = m->x; k.rows = K; k.in = H; k.dtype = L.egd; k.w = L.eg; k.out = FI;
    k.y = m->gate; k.mode = m->mode; k.ids = m->ids; k.stride = L.eg_stride; k.x_per_slot = 0;
    k.nexp = (int)E; k.bias = L.egb; k.w2 = L.eu; k.bias2 = L.eub; k.alpha = d.swiglu_alpha;
    k.limit = d.swiglu_limit; k.nw = L.post_norm; k.eps = d.rms_eps;
    if (self_route) {
      k.rl = m->route; k.rw = m->rw; k.rexp = (int)E; k.rk = (int)K; k.rnorm = d.norm_topk;
    }
    if ((rc = enqueue_linear(m->c, k))) return rc;
    LinearCall dn;
    dn.x = m->gate; dn.rows = K; dn.in = FI; dn.dtype = L.edd; dn.w = L.ed; dn.out = H;
    dn.y = m->x; dn.res = m->x; dn.cw = m->rw; dn.mode = m->mode; dn.ids = m->ids;
    dn.stride = L.ed_stride; dn.x_per_slot = 1; dn.nexp = (int)E; dn.bias = L.edb;
    if ((rc = enqueue_linear(m->c, dn))) return rc;
  }
  return 0;
}

// the layers of one chunk of n rows at positions past.., x holding the
// embeddings; leaves h = the final norm of x. graph: the position is read
// from m->pos (decode step under capture)
static int layers(ihip_model* m, int64_t n, int64_t past, bool graph)
{
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd,
                kvw = (int64_t)d.kv_heads * hd;
  // one row (decode): every GEMV quantizes its activation row in registers;
  // a chunk: the rows are quantized once per activation buffer
  const bool one = n == 1;
  if (one && one_row_fused(m)) return layers_one(m, past, graph);
  int rc = ihip_enqueue_rmsnorm(m->c, m->x, m->L[0].input_norm, m->h, n, H, d.rms_eps);
  if (rc) return rc;
  for (int l = 0; l < d.layers; l++) {
    const DevLayer& L = m->L[l];
    QCache qh{m->xq0, m->xqk};
    QCache* qhp = one ? nullptr : &qh;
    // attention block (decoder.pas:2625-2702)
    if ((rc = lin(m, m->h, qhp, n, H, L.qd, L.q, qw, L.qb, m->q))) return rc;
    if ((rc = lin(m, m->h, qhp, n, H, L.kd, L.k, kvw, L.kb, m->k))) return rc;
    if ((rc = lin(m, m->h, qhp, n, H, L.vd, L.v, kvw, L.vb, m->v))) return rc;
    if ((rc = rope_attn(m, L, n, past, graph))) return rc;
    QCache qa{m->xq0, m->xqk};
    if ((rc = lin(m, m->attn, one ? nullptr : &qa, n, qw, L.od, L.o, H, L.ob, m->tmp))) return rc;
    // residual, then the pre-FFN norm
    if ((rc = ihip_enqueue_addnorm(m->c, m->x, m->tmp, L.post_norm, m->h, n, H, d.rms_eps)))
      return rc;
    QCache qf{m->xq0, m->xqk};
    QCache* qfp = one ? nullptr : &qf;
    bool moe_out = false;  // the FFN output is the expert rows (added by the next norm)
    if (!L.moe) {
      // DenseFfn (decoder.pas:2866-2878)
      const int64_t F = d.ffn;
      if (one) {
        // gate, up and SwiGLU in one pass
        LinearCall k;
        k.x = m->h; k.rows = 1; k.in = H; k.dtype = L.gd; k.w = L.gate; k.out = F;
        k.y = m->gate; k.mode = m->mode; k.w2 = L.up; k.alpha = d.swiglu_alpha;
        k.limit = d.swiglu_limit;
        if (L.gd != L.ud) return fail(IHIP_E_ARG, "model: gate and up of one type");
        if ((rc = enqueue_linear(m->c, k))) return rc;
      } else {
        if ((rc = lin(m, m->h, qfp, n, H, L.gd, L.gate, F, 0, m->gate))) return rc;
        if ((rc = lin(m, m->h, qfp, n, H, L.ud, L.up, F, 0, m->up))) return rc;
        if ((rc = ihip_enqueue_swiglu(m->c, m->gate, m->up, n * F, d.swiglu_alpha,
                                      d.swiglu_limit)))
          return rc;
      }
      QCache qg{m->xqf, m->xqf};
      if ((rc = lin(m, m->gate, one ? nullptr : &qg, n, F, L.dd, L.down, H, 0, m->tmp))) return rc;
    } else {
      // MoeBlock (decoder.pas:3037-3053) with the experts chosen on the
      // device (model.qwen3.cuda.pas:1152-1205)
      const int64_t E = d.experts, K = d.experts_used, FI = d.expert_ffn;
      if ((rc = lin(m, m->h, qfp, n, H, L.rd, L.router, E, L.router_b, m->route))) return rc;
      struct {
        const float* logits;
        int* ids;
        float* w;
        int32_t experts, k, norm, rows;
      } ra = {(const float*)m->route, (int*)m->ids, (float*)m->rw, (int32_t)E, (int32_t)K,
              d.norm_topk, (int32_t)n};
      if ((rc = launch(m->c, "route", dim3((unsigned)n), dim3(256), &ra))) return rc;
      if (one) {
        // the token's K experts: gate, up and SwiGLU in one pass per slot,
        // then down per slot; the weighted sum goes into the next norm
        LinearCall k;
        k.x = m->h; k.rows = K; k.in = H; k.dtype = L.egd; k.w = L.eg; k.out = FI;
        k.y = m->gate; k.mode = m->mode; k.ids = m->ids; k.stride = L.eg_stride; k.x_per_slot = 0;
        k.nexp = (int)E; k.bias = L.egb; k.w2 = L.eu; k.bias2 = L.eub; k.alpha = d.swiglu_alpha;
        k.limit = d.swiglu_limit;
        if ((rc = enqueue_linear(m->c, k))) return rc;
        LinearCall dn;
        dn.x = m->gate; dn.rows = K; dn.in = FI; dn.dtype = L.edd; dn.w = L.ed; dn.out = H;
        dn.y = m->eout; dn.mode = m->mode; dn.ids = m->ids; dn.stride = L.ed_stride;
        dn.x_per_slot = 1; dn.nexp = (int)E; dn.bias = L.edb;
        if ((rc = enqueue_linear(m->c, dn))) return rc;
      } else {
        struct {
          const int* ids;
          int* perm;
          void* items;
          int32_t slots, experts, max_items, chunk;
        } pa = {(const int*)m->ids, (int*)m->perm, (void*)m->items, (int32_t)(n * K), (int32_t)E,
                (int32_t)((n * K + m->item_rows - 1) / m->item_rows + E), m->item_rows};
        if ((rc = launch(m->c, "moe_plan", dim3(1), dim3(256), &pa))) return rc;
        // gate and up: slot s = row s / K, expert ids[s], grouped by expert
        bool q0 = false;
        if (m->mode == IHIP_MODE_Q8 && q8_kind(L.egd) >= 0) {
          bool& hv = q8_kind(L.egd) ? qf.havek : qf.have0;
          uint64_t buf = q8_kind(L.egd) ? qf.bufk : qf.buf0;
          if (!hv) {
            if ((rc = enqueue_quantize(m->c, m->h, n, H, q8_kind(L.egd), buf))) return rc;
            hv = true;
          }
          q0 = true;
        }
        uint64_t xqg = q8_kind(L.egd) == 1 ? qf.bufk : qf.buf0;
        if ((rc = lin_ids(m, m->h, xqg, n, H, L.egd, L.eg, L.eg_stride, FI, m->ids, n * K, (int)K,
                          L.egb, m->gate, q0)))
          return rc;
        bool qu = q0 && q8_kind(L.eud) == q8_kind(L.egd);
        uint64_t xqu = q8_kind(L.eud) == 1 ? qf.bufk : qf.buf0;
        if ((rc = lin_ids(m, m->h, xqu, n, H, L.eud, L.eu, L.eg_stride, FI, m->ids, n * K, (int)K,
                          L.eub, m->up, qu)))
          return rc;
        if ((rc = ihip_enqueue_swiglu(m->c, m->gate, m->up, n * K * FI, d.swiglu_alpha,
                                      d.swiglu_limit)))
          return rc;
        if ((rc = lin_ids(m, m->gate, m->xqf, n * K, FI, L.edd, L.ed, L.ed_stride, H, m->ids,
                          n * K, 1, L.edb, m->eout, false)))
          return rc;
      }
      moe_out = true;
    }
    // residual, then the next layer's input norm (or the final norm)
    uint64_t nw = l + 1 < d.layers ? m->L[l + 1].input_norm : m->final_norm;
    if (moe_out)
      rc = enqueue_addnorm_moe(m->c, m->x, m->eout, m->rw, d.experts_used, nw, m->h, n, H, d.rms_eps);
    else
      rc = ihip_enqueue_addnorm(m->c, m->x, m->tmp, nw, m->h, n, H, d.rms_eps);
    if (rc) return rc;
  }
  return 0;
}

static int head(ihip_model* m, int64_t n, bool all, uint64_t y)
{
  const ihip_model_desc& d = m->d;
  QCache qh{m->xq0, m->xqk};
  if (n == 1 && one_row_fused(m)) {
    // layers_one left the residual: the final norm is staged by the head
    LinearCall k;
    k.x = m->x; k.rows = 1; k.in = d.hidden; k.dtype = m->head_dt; k.w = m->head;
    k.out = d.vocab; k.y = y; k.mode = m->mode; k.nw = m->final_norm; k.eps = d.rms_eps;
    return enqueue_linear(m->c, k);
  }
  if (all) return lin(m, m->h, &qh, n, d.hidden, m->head_dt, m->head, d.vocab, 0, y);
  return lin(m, m->h + (uint64_t)(n - 1) * d.hidden * 4, nullptr, 1, d.hidden, m->head_dt,
             m->head, d.vocab, 0, y);
}

// one chunk: ids and cos/sin uploaded, embeddings, layers, head
static int chunk(ihip_model* m, const int32_t* ids, int64_t n, bool want_logits, bool all,
                 uint64_t logits_dev)
{
  const ihip_model_desc& d = m->d;
  std::vector<float> cs((size_t)n * d.head_dim);
  rotary(d, m->length, n, cs.data());
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)m->tok, (void*)ids, n * 4, m->c->stream));
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)m->cs, cs.data(), cs.size() * 4, m->c->stream));
  int rc = ihip_enqueue_embed(m->c, m->embed, m->embed_dt, d.vocab, d.hidden, m->tok, n, m->x);
  if (!rc) rc = layers(m, n, m->length, false);
  if (!rc && want_logits) rc = head(m, n, all, logits_dev);
  // the host vectors must outlive the copies
  IHIP_CHECK(hipStreamSynchronize(m->c->stream));
  if (!rc) m->length += n;
  return rc;
}

// the next id from the logits: the argmax, or a draw of the sampler
static int next_token(ihip_model* m)
{
  return m->sampler ? ihip_enqueue_sample(m->c, m->sampler, m->logits, m->d.vocab, m->next)
                    : ihip_enqueue_argmax(m->c, m->logits, m->d.vocab, m->next);
}

// the decode step as a graph: embed(tok) -> layers(pos) -> head -> next id
static int decode_body(ihip_model* m)
{
  ihip_ctx* c = m->c;
  int rc = ihip_enqueue_embed(c, m->embed, m->embed_dt, m->d.vocab, m->d.hidden, m->tok, 1, m->x);
  if (!rc) rc = layers(m, 1, 0, true);
  if (!rc) rc = head(m, 1, false, m->logits);
  if (!rc) rc = next_token(m);
  return rc;
}

static int decode_graph(ihip_model* m)
{
  ihip_ctx* c = m->c;
  int rc = ihip_capture_begin(c);
  if (rc) return rc;
  rc = decode_body(m);
  int rc2 = ihip_capture_end(c, 0);
  if (rc) return rc;
  if (rc2) return rc2;
  m->graph_ready = true;
  c->slot_owner[0] = m;
  return 0;
}

// steps decode steps from token `first` (not yet in the cache): each one
// graph launch that writes the next id; out_ids[i] the id after step i
static int decode_steps(ihip_model* m, int32_t first, int64_t steps, int32_t* out_ids)
{
  ihip_ctx* c = m->c;
  int rc = 0;
  // slot 0 holds one model's decode graph: another model of this context
  // may have captured into it since
  if (m->use_graphs && (!m->graph_ready || c->slot_owner[0] != m) && (rc = decode_graph(m))) return rc;
  std::vector<float> cs(m->d.head_dim);
  int32_t tok = first;
  for (int64_t i = 0; i < steps; i++) {
    int32_t pos = (int32_t)m->length;
    rotary(m->d, pos, 1, cs.data());
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)m->tok, &tok, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)m->pos, &pos, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)m->cs, cs.data(), cs.size() * 4, c->stream));
    if ((rc = m->use_graphs ? ihip_graph_launch(c, 0) : decode_body(m))) return rc;
    IHIP_CHECK(hipMemcpyDtoHAsync(&out_ids[i], (hipDeviceptr_t)m->next, 4, c->stream));
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    m->length++;
    tok = out_ids[i];
  }
  return 0;
}

}  // namespace ihip

using namespace ihip;

extern "C" {

int ihip_model_rotary(const ihip_model_desc* d, int64_t first, int64_t rows, float* cs)
{
  if (!d || !cs || rows < 1 || d->head_dim < 2) return fail(IHIP_E_ARG, "ihip_model_rotary");
  rotary(*d, first, rows, cs);
  return 0;
}

int ihip_model_create(ihip_ctx* c, const ihip_model_desc* desc, int mode, int kv_f16,
                      int64_t max_tokens, ihip_model** out)
{
  if (!c || !desc || !out || !desc->layer || desc->layers < 1 || max_tokens < 1)
    return fail(IHIP_E_ARG, "ihip_model_create");
  *out = nullptr;
  ihip_model* m = new ihip_model();
  m->c = c;
  m->d = *desc;
  m->layer_desc.assign(desc->layer, desc->layer + desc->layers);
  m->d.layer = m->layer_desc.data();
  m->mode = mode;
  m->kv_f16 = kv_f16;
  m->max_tokens = max_tokens;
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd,
                kvw = (int64_t)d.kv_heads * hd;
  int rc = 0;
  auto bad = [&](int r) {
    ihip_model_destroy(m);
    return r;
  };
  // UploadWeights (model.qwen3.cuda.pas:602-828)
  if ((rc = upw(m, d.embed, d.vocab, H, 1, m->embed, m->embed_dt))) return bad(rc);
  if (d.head.data) {
    if ((rc = upw(m, d.head, d.vocab, H, 1, m->head, m->head_dt))) return bad(rc);
  } else {
    m->head = m->embed;
    m->head_dt = m->embed_dt;
  }
  if ((rc = upf(m, d.final_norm, H, m->final_norm))) return bad(rc);
  m->L.resize(d.layers);
  bool any_moe = false;
  for (int l = 0; l < d.layers; l++) {
    const ihip_layer_desc& s = m->layer_desc[l];
    DevLayer& L = m->L[l];
    L.window = s.window;
    L.moe = s.moe;
    any_moe |= s.moe != 0;
    if ((rc = upf(m, s.input_norm, H, L.input_norm)) || (rc = upf(m, s.post_norm, H, L.post_norm)) ||
        (rc = upw(m, s.q, qw, H, 1, L.q, L.qd)) || (rc = upw(m, s.k, kvw, H, 1, L.k, L.kd)) ||
        (rc = upw(m, s.v, kvw, H, 1, L.v, L.vd)) || (rc = upw(m, s.o, H, qw, 1, L.o, L.od)) ||
        (rc = upf(m, s.q_bias, qw, L.qb)) || (rc = upf(m, s.k_bias, kvw, L.kb)) ||
        (rc = upf(m, s.v_bias, kvw, L.vb)) || (rc = upf(m, s.o_bias, H, L.ob)) ||
        (rc = upf(m, s.q_norm, hd, L.qn)) || (rc = upf(m, s.k_norm, hd, L.kn)) ||
        (rc = upf(m, s.sinks, d.heads, L.sinks)))
      return bad(rc);
    if (!s.moe) {
      if ((rc = upw(m, s.gate, d.ffn, H, 1, L.gate, L.gd)) || (rc = upw(m, s.up, d.ffn, H, 1, L.up, L.ud)) ||
          (rc = upw(m, s.down, H, d.ffn, 1, L.down, L.dd)))
        return bad(rc);
    } else {
      const int64_t E = d.experts, FI = d.expert_ffn;
      if ((rc = upw(m, s.router, E, H, 1, L.router, L.rd)) || (rc = upf(m, s.router_bias, E, L.router_b)) ||
          (rc = upw(m, s.exp_gate, FI, H, E, L.eg, L.egd)) ||
          (rc = upw(m, s.exp_up, FI, H, E, L.eu, L.eud)) ||
          (rc = upw(m, s.exp_down, H, FI, E, L.ed, L.edd)) ||
          (rc = upf(m, s.exp_gate_bias, E * FI, L.egb)) ||
          (rc = upf(m, s.exp_up_bias, E * FI, L.eub)) ||
          (rc = upf(m, s.exp_down_bias, E * H, L.edb)))
        return bad(rc);
      if (L.egd != L.eud) return bad(fail(IHIP_E_ARG, "experts: gate and up of one type"));
      L.eg_stride = (int64_t)row_bytes(L.egd, H) * FI;
      L.ed_stride = (int64_t)row_bytes(L.edd, FI) * H;
    }
    const uint64_t kvbytes = (uint64_t)max_tokens * kvw * (kv_f16 ? 2 : 4);
    if ((rc = dalloc(m, kvbytes, L.kc)) || (rc = dalloc(m, kvbytes, L.vc))) return bad(rc);
  }
  // activations of one chunk
  const int64_t N = CHUNK;
  int64_t F = std::max<int64_t>(d.ffn, 1);
  int64_t EK = any_moe ? (int64_t)d.experts_used * d.expert_ffn : 0;
  int64_t wide = std::max<int64_t>({F, EK, qw, H, (int64_t)d.experts});
  if ((rc = dalloc(m, N * H * 4, m->x)) || (rc = dalloc(m, N * H * 4, m->h)) ||
      (rc = dalloc(m, N * H * 4, m->tmp)) || (rc = dalloc(m, N * qw * 4, m->q)) ||
      (rc = dalloc(m, N * kvw * 4, m->k)) || (rc = dalloc(m, N * kvw * 4, m->v)) ||
      (rc = dalloc(m, N * qw * 4, m->attn)) || (rc = dalloc(m, N * wide * 4, m->gate)) ||
      (rc = dalloc(m, N * wide * 4, m->up)) ||
      (rc = dalloc(m, N * std::max<int64_t>(d.experts, 1) * 4, m->route)) ||
      (rc = dalloc(m, N * std::max(d.experts_used, 1) * 4, m->ids)) ||
      (rc = dalloc(m, N * std::max(d.experts_used, 1) * 4, m->rw)) ||
      (rc = dalloc(m, N * std::max(d.experts_used, 1) * H * 4, m->eout)) ||
      (rc = dalloc(m, N * hd * 4, m->cs)) || (rc = dalloc(m, N * 4, m->tok)) ||
      (rc = dalloc(m, (uint64_t)d.vocab * 4, m->logits)) || (rc = dalloc(m, 256, m->next)) ||
      (rc = dalloc(m, 256, m->pos)) ||
      (rc = dalloc(m, N * std::max(d.experts_used, 1) * 4, m->perm)) ||
      (rc = dalloc(m, (N * std::max(d.experts_used, 1) / 8 + 1 + std::max(d.experts, 1)) * 16,
                   m->items)))
    return bad(rc);
  if (hd % 8 || hd > 256) return bad(fail(IHIP_E_ARG, "model: head size not a multiple of 8 up to 256"));
  if ((rc = dalloc(m, 256 * 128, m->done))) return bad(rc);
  {
    const hipError_t e = hipMemsetAsync((void*)m->done, 0, 256 * 128, m->c->stream);
    if (e != hipSuccess) return bad(hip_fail(e, "model: counters"));
  }
  if ((rc = dalloc(m, (uint64_t)d.heads * N * attention_splits(max_tokens) * (hd + 2) * 8,
                   m->attn_part)))
    return bad(rc);
  // moe_plan counts the slots per expert in LDS (4096 experts); a chunk's
  // work items stay within one grid dimension
  if (any_moe && (d.experts > 4096 || N * d.experts_used > 65535))
    return bad(fail(IHIP_E_ARG, "model: more than 4096 experts or 65535 slots per chunk"));
  // a prompt chunk's experts on the MFMA GEMM when every expert matrix can
  // run there: work items of 64 slots
  bool all_gemm = any_moe;
  for (const DevLayer& L : m->L)
    if (L.moe)
      all_gemm = all_gemm && gemm_runs(c, L.egd, mode) && gemm_runs(c, L.eud, mode) &&
                 gemm_runs(c, L.edd, mode);
  m->item_rows = all_gemm ? 64 : 8;
  const uint64_t qin = std::max<int64_t>({H, qw, F, (int64_t)d.expert_ffn});
  const uint64_t qrow = qin + 4 * (qin / 32);
  if ((rc = dalloc(m, N * qrow, m->xq0)) || (rc = dalloc(m, N * qrow, m->xqk)) ||
      (rc = dalloc(m, N * std::max(d.experts_used, 1) * qrow, m->xqf)))
    return bad(rc);
  *out = m;
  return 0;
}

void ihip_model_destroy(ihip_model* m)
{
  if (!m) return;
  (void)hipStreamSynchronize(m->c->stream);
  for (auto p : m->owned) (void)hipFree((void*)p);
  if (m->logits_all) (void)hipFree((void*)m->logits_all);
  ihip_sampler_destroy(m->sampler);
  for (auto& u : m->uploaded) ihip_forget_weights(m->c, u.first, u.first + u.second);
  if (m->c->slot_owner[0] == m) m->c->slot_owner[0] = nullptr;
  delete m;
}

int ihip_model_reset(ihip_model* m)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_reset");
  m->length = 0;
  return 0;
}

int ihip_model_forward(ihip_model* m, const int32_t* ids, int64_t count, float* logits,
                       int all_logits)
{
  if (!m || !ids || count < 1) return fail(IHIP_E_ARG, "ihip_model_forward: no tokens");
  if (m->length + count > m->max_tokens)
    return fail(IHIP_E_ARG, "ihip_model_forward: beyond the KV cache");
  for (int64_t i = 0; i < count; i++)
    if (ids[i] < 0 || ids[i] >= m->d.vocab) return fail(IHIP_E_ARG, "token id outside the vocabulary");
  std::lock_guard<std::mutex> g(m->c->lock);
  for (int64_t s = 0; s < count; s += m->chunk_rows) {
    int64_t n = std::min(m->chunk_rows, count - s);
    bool last = s + n == count;
    bool want = logits && (all_logits || last);
    uint64_t ldev = m->logits;
    if (want && all_logits) {
      if (m->logits_all_rows < n) {
        if (m->logits_all) (void)hipFree((void*)m->logits_all);
        void* p = nullptr;
        IHIP_CHECK(hipMalloc(&p, (uint64_t)CHUNK * m->d.vocab * 4));
        m->logits_all = (uint64_t)p;
        m->logits_all_rows = CHUNK;
      }
      ldev = m->logits_all;
    }
    int rc = chunk(m, ids + s, n, want, all_logits != 0, ldev);
    if (rc) return rc;
    if (want) {
      float* dst = all_logits ? logits + s * m->d.vocab : logits;
      uint64_t rows = all_logits ? n : 1;
      IHIP_CHECK(hipMemcpyDtoHAsync(dst, (hipDeviceptr_t)ldev, rows * m->d.vocab * 4, m->c->stream));
      IHIP_CHECK(hipStreamSynchronize(m->c->stream));
    }
  }
  return 0;
}

int ihip_model_greedy(ihip_model* m, const int32_t* prompt, int64_t n, int64_t max_new,
                      int32_t* out_ids)
{
  if (!m || !prompt || n < 1 || max_new < 1 || !out_ids) return fail(IHIP_E_ARG, "ihip_model_greedy");
  if (m->length + n + max_new > m->max_tokens)
    return fail(IHIP_E_ARG, "ihip_model_greedy: beyond the KV cache");
  ihip_ctx* c = m->c;
  auto t0 = std::chrono::steady_clock::now();
  int rc = 0;
  {
    // the prompt: every chunk, logits of the last row only, argmax on device
    std::lock_guard<std::mutex> g(c->lock);
    for (int64_t s = 0; s < n && !rc; s += m->chunk_rows) {
      int64_t k = std::min(m->chunk_rows, n - s);
      rc = chunk(m, prompt + s, k, s + k == n, false, m->logits);
    }
    if (!rc) rc = next_token(m);
    if (!rc) {
      IHIP_CHECK(hipMemcpyDtoHAsync(&out_ids[0], (hipDeviceptr_t)m->next, 4, c->stream));
      IHIP_CHECK(hipStreamSynchronize(c->stream));
    }
  }
  if (rc) return rc;
  auto t1 = std::chrono::steady_clock::now();
  std::lock_guard<std::mutex> g(c->lock);
  // the new ids, then the last one into the cache too (TDecoderModel.Greedy:
  // a Forward without logits after the last step), through the same graph
  if (max_new > 1 && (rc = decode_steps(m, out_ids[0], max_new - 1, out_ids + 1))) return rc;
  int32_t spare;
  if ((rc = decode_steps(m, out_ids[max_new - 1], 1, &spare))) return rc;
  auto t2 = std::chrono::steady_clock::now();
  m->prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  m->decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  return 0;
}

int ihip_model_decode(ihip_model* m, int32_t first, int64_t steps, int32_t* out_ids)
{
  if (!m || steps < 1 || !out_ids || first < 0 || first >= m->d.vocab)
    return fail(IHIP_E_ARG, "ihip_model_decode");
  if (m->length + steps > m->max_tokens) return fail(IHIP_E_ARG, "ihip_model_decode: beyond the KV cache");
  std::lock_guard<std::mutex> g(m->c->lock);
  auto t0 = std::chrono::steady_clock::now();
  int rc = decode_steps(m, first, steps, out_ids);
  m->decode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  return rc;
}

int ihip_model_chunk(ihip_model* m, int64_t rows)
{
  if (!m || rows < 1 || rows > CHUNK) return fail(IHIP_E_ARG, "ihip_model_chunk: 1.." + std::to_string(CHUNK) + " rows");
  m->chunk_rows = rows;
  return 0;
}

int ihip_model_sampling(ihip_model* m, const ihip_sampling* s)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_sampling");
  std::lock_guard<std::mutex> g(m->c->lock);
  ihip_sampler* k = nullptr;
  if (s && s->temperature > 0) {
    int rc = ihip_sampler_create(m->c, s, m->d.vocab, &k);
    if (rc) return rc;
  } else if (s) {
    // greedy: the settings are still checked as TInferSampler.Create does
    ihip_sampling chk = *s;
    chk.temperature = 0;
    ihip_sampler* probe = nullptr;
    int rc = ihip_sampler_create(m->c, &chk, 1, &probe);
    ihip_sampler_destroy(probe);
    if (rc) return rc;
  }
  ihip_sampler_destroy(m->sampler);
  m->sampler = k;
  m->graph_ready = false;  // the decode graph is captured again with it
  return 0;
}

int ihip_model_use_graphs(ihip_model* m, int on)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_use_graphs");
  m->use_graphs = on != 0;
  return 0;
}

int ihip_model_timing(ihip_model* m, double* prefill_ms, double* decode_ms)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_timing");
  if (prefill_ms) *prefill_ms = m->prefill_ms;
  if (decode_ms) *decode_ms = m->decode_ms;
  return 0;
}

}  // extern "C"
