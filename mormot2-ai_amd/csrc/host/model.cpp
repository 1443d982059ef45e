// model.cpp - TQwen3Cuda of the reference
// (src/infer/mormot.ai.infer.model.qwen3.cuda.pas:150-1761) for HIP: the
// whole decoder on the device behind TDecoderDevice (decoder.pas:907-928).
// Qwen3 dense, Qwen3-MoE and gpt-oss shapes: per-head q/k norms, biases,
// sinks, sliding windows, clamped SwiGLU, experts chosen on the device;
// Qwen3.5: Gated DeltaNet layers with their states per context, the output
// gate of the attention and a partial rotary share. Gemma 4: heads of their
// own shape per layer, K=V, the value norm, a second rotary set, the norms
// around both blocks, GeGLU, the dense block beside the experts (expert
// scales, experts stored gate-and-up in one tensor), the layer scalar, the
// embedding scale and the logit softcap.
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
#include <memory>

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
  int window = 0, moe = 0;
  // Qwen3.5: the mixer and the output gate; a DeltaNet layer's weights
  int mixer = IHIP_MIXER_ATTENTION, output_gate = 0;
  uint64_t lqkv = 0, lz = 0, lb = 0, la = 0, lout = 0, lconv = 0, ldt = 0, lnega = 0, lnorm = 0;
  int lqkvd = 0, lzd = 0, lbd = 0, lad = 0, loutd = 0;
  uint64_t lba = 0;  // beta's rows, then alpha's, as one matrix (types alike), for the one-row path
  int lbad = 0;
  // Gemma 4: this layer's heads, K=V, the rotary set; the norms around the
  // blocks, those of the dense block beside the experts, the expert scales
  // and the layer scalar (0: none)
  int64_t hd = 0, kvh = 0;
  int k_is_v = 0, rope_set = 0;
  int no_rope = 0;  // no rotary positions on q and k (NoPE): the kernels get no rotary table
  uint64_t attn_out_norm = 0, ffn_out_norm = 0, dense_out_norm = 0, moe_in_norm = 0, moe_out_norm = 0;
  uint64_t router_norm = 0, expert_scale = 0, scalar = 0;
};

}  // namespace ihip

// a context of a model on the device (TQwen3CuContext,
// model.qwen3.cuda.pas:150-198): its KV cache, which grows as tokens come
// (Prepare, :856-940), the activations of one chunk, the id of every cached
// position and its own decode graph
struct ihip_mctx {
  ihip_model* m = nullptr;
  int64_t capacity = 0, length = 0;
  std::vector<int32_t> ids;         // the token of each cached position, -1: an embedding row
  std::vector<uint64_t> kc, vc;     // per layer [capacity, kvw] (f16 or f32)
  // activations for CHUNK rows
  uint64_t x = 0, h = 0, tmp = 0, q = 0, k = 0, v = 0, attn = 0, gate = 0, up = 0;
  uint64_t route = 0, ids_dev = 0, rw = 0, eout = 0, cs = 0, tok = 0, logits = 0, next = 0, pos = 0;
  uint64_t xq0 = 0, xqk = 0, xqf = 0;  // quantized h (Q8_0, Q8_K) and FFN input
  uint64_t perm = 0, items = 0;         // the experts of a prompt chunk (moe_plan)
  uint64_t attn_part = 0, attn_part_bytes = 0;  // flash-decoding partials
  // Qwen3.5: per DeltaNet layer its convolution inputs and state S (zero when
  // a sequence starts); the chunk's DeltaNet channels, gates, beta, decay and
  // the rule's output; a gated attention's query+gate rows and its gates
  std::vector<uint64_t> conv, state;
  uint64_t qkv = 0, z = 0, beta = 0, decay = 0, core = 0, qg = 0, gq = 0;
  // Gemma 4: the second rotary set's cos/sin, the experts' sum of a row
  uint64_t cs2 = 0, moe = 0;
  // the rotary rows of positions 0 .. cs_rows - 1 (cs_cap allocated), and the
  // second set's: the decode graph's last launch takes the next position's
  // rows from them
  uint64_t cs_tab = 0, cs2_tab = 0;
  int64_t cs_rows = 0, cs_cap = 0;
  // pinned staging of the ids of a pipelined decode
  int32_t* ids_pinned = nullptr;
  int64_t ids_pinned_n = 0;
  // the restore points of the DeltaNet states (TDecoderContext.CheckpointId,
  // MaxCheckpoints, decoder.pas:466-620, :1049-1230): the states before the
  // CheckpointId tokens of aligned parts, the oldest first; each in a slot of
  // per-layer copies of conv and state
  int32_t ckpt_id = -1;
  int64_t ckpt_max = 4;     // DECODER_CHECKPOINTS (decoder.pas:305)
  bool aligned = true;      // the cached rows were split as a fresh pass splits them
  bool state_ok = true;     // false while (or after a failure of) a forward
  std::vector<std::pair<int64_t, int>> ckpts;  // (length, slot)
  std::vector<std::vector<uint64_t>> slot_conv, slot_state;
  // zeroed counters of the decode attention's heads (the last range block of
  // a head merges the head)
  uint64_t done = 0;
  uint64_t logits_all = 0;
  int64_t logits_all_rows = 0;
  std::vector<uint64_t> owned;
  // the decode step's graph (one per context: it holds this context's
  // buffers), captured for a capacity and a sampler
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool graph_ready = false;
  int64_t graph_capacity = 0;
  int graph_sampler = -1;
  // the rows of the logits a draw considers (0: the vocabulary; NativeDecode
  // draws among the ids its tokenizer has), and the count the graph holds
  int64_t draw_ids = 0, graph_draw = -1;
  double prefill_ms = 0, decode_ms = 0;
  bool is_default = false;  // the model's own context (ihip_model_*), freed with it
};

struct ihip_model {
  ihip_ctx* c = nullptr;
  ihip_model_desc d{};
  std::vector<ihip_layer_desc> layer_desc;
  std::vector<ihip::DevLayer> L;
  int mode = IHIP_MODE_Q8, kv_f16 = 0;
  uint64_t embed = 0, final_norm = 0, head = 0;
  int embed_dt = 0, head_dt = 0;
  bool any_moe = false;
  bool recurrent = false;  // a DeltaNet layer: the context carries states
  bool gated = false;      // an attention layer with an output gate
  bool gemma = false;      // Gemma 4's settings: no fused one-row path
  // the widest heads of any layer, and the heads of the second rotary set
  int64_t max_qw = 0, max_kvw = 0, max_hd = 0, hd2 = 0;
  // the host ranges of the uploaded weights: forgotten when the model goes,
  // as a model does in its destructor (backend.pas:151-158) - new host
  // tensors at a reused address must not meet the stale device copy
  std::vector<std::pair<const uint8_t*, uint64_t>> uploaded;
  // host copies the model made for an upload (a DeltaNet's beta and alpha
  // rows as one matrix): kept while their device copies are cached
  std::vector<std::unique_ptr<std::vector<uint8_t>>> host_owned;
  ihip_sampler* sampler = nullptr;  // null: the argmax
  int sampler_epoch = 0;            // bumped by ihip_model_sampling (graphs captured again)
  bool use_graphs = true;  // TQwen3Cuda.UseGraphs (model.qwen3.cuda.pas:253-262)
  // CheckRoute (model.qwen3.cuda.pas:288-300): after every one-row route on
  // the device the step waits and compares the choice with the host's Route
  bool check_route = false;
  // a test's capture of the residual rows after one layer of a chunk
  float* dbg_host = nullptr;
  int dbg_layer = -1;
  int64_t route_checks = 0, route_mismatches = 0;
  double route_max_diff = 0;
  // TDecoderRouteTape replayed (decoder.pas:2993-3035): the picks and
  // weights of another run (the CPU's), given to every routed row in turn in
  // place of the device's own; the device's own choice counted where it
  // differs, with the largest router gap of such a row
  std::vector<int32_t> tape_ids;
  std::vector<float> tape_w;
  int64_t tape_rows = 0, tape_pos = 0, tape_routes = 0, tape_differs = 0;
  double tape_gap = 0;
  int64_t chunk_rows = ihip::CHUNK;  // prompt rows per chunk (ihip_model_chunk), at most CHUNK
  int item_rows = 8;  // slots per grouped-expert work item: 64 when the experts run on the GEMM
  ihip_mctx* def = nullptr;  // the context of the ihip_model_* calls
  std::vector<ihip_mctx*> contexts;  // every live context (freed with the model)
};

namespace ihip {

// decoder.pas:1735-1741 and 1759-1829: inverse frequencies, every step
// rounded to single as the reference's float32 tensors; YaRN when factor > 0
// the rotating values of a head (RopeDims): the whole head unless given
static int64_t rope_dims(const ihip_model_desc& d) { return d.rope_dims > 0 ? d.rope_dims : d.head_dim; }

static void inv_freq(const ihip_model_desc& d, std::vector<float>& f, float& scale)
{
  const int64_t dim = rope_dims(d), half = dim / 2;
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
// sin rounded to single, then times the YaRN scale in single; [rows, rot / 2]
// cos, then sin
static void rotary(const ihip_model_desc& d, int64_t first, int64_t rows, float* cs)
{
  std::vector<float> f;
  float rs;
  inv_freq(d, f, rs);
  const int64_t half = rope_dims(d) / 2;
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

// TDecoderModel.Rotary2 (decoder.pas:1742-1752, :2524-2537): the second
// set over heads of hd2, 1 / theta2 ^ (2i / hd2) (each step rounded to
// single) for the first rope2_pairs pairs, frequency 0 for the others; no
// YaRN scale
static void rotary2(const ihip_model_desc& d, int64_t hd2, int64_t first, int64_t rows, float* cs)
{
  const int64_t half = hd2 / 2;
  const double lt = std::log(d.rope2_theta);
  std::vector<float> f(half, 0.f);
  for (int64_t i = 0; i < half && i < d.rope2_pairs; i++) {
    float e = (float)((double)(2 * i) / (double)hd2);
    float p = (float)std::exp(lt * (double)e);
    f[i] = 1.0f / p;
  }
  float* sn = cs + rows * half;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < half; i++) {
      float angle = f[i] * (float)(first + r);
      cs[r * half + i] = (float)std::cos((double)angle);
      sn[r * half + i] = (float)std::sin((double)angle);
    }
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

static int lin(ihip_mctx* s, uint64_t x, QCache* qc, int64_t rows, int64_t in, int dt,
               uint64_t w, int64_t out, uint64_t bias, uint64_t y)
{
  ihip_model* m = s->m;
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

static int lin_ids(ihip_mctx* s, uint64_t x, uint64_t xqbuf, int64_t xrows, int64_t in, int dt,
                   uint64_t w, int64_t stride, int64_t out, uint64_t ids, int64_t slots,
                   int x_div, uint64_t bias, uint64_t y, bool quantized)
{
  ihip_model* m = s->m;
  LinearCall k;
  k.x = x; k.rows = slots; k.in = in; k.dtype = dt; k.w = w; k.out = out; k.bias = bias;
  k.y = y; k.mode = m->mode; k.ids = ids; k.stride = stride; k.x_per_slot = x_div;
  k.nexp = m->d.experts;
  if (slots > m->d.experts_used) {
    // a prompt chunk: the slots grouped by expert (moe_plan), up to
    // item_rows rows per work item (8 for the 8-row GEMV, 64 for the GEMM),
    // so an expert's matrix is read once per that many of its tokens
    k.ids = 0;
    k.items = s->items;
    k.perm = s->perm;
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

static int rope_attn(ihip_mctx* s, int l, int64_t n, int64_t past, bool graph)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const DevLayer& L = m->L[l];
  const int64_t hd = L.hd, kvh = L.kvh;
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
    int32_t rows, heads, kvh, hd, past, f16, rot, vnorm;
  } ra = {(float*)s->q, (const float*)s->k,
          // K=V: the values are the raw keys (normed by ValueNorm, not rotated)
          (const float*)(L.k_is_v ? s->k : s->v), (const float*)L.qn, (const float*)L.kn,
          (const float*)(L.no_rope ? 0 : L.rope_set ? s->cs2 : s->cs), (void*)s->kc[l], (void*)s->vc[l],
          graph ? (const int*)s->pos : nullptr, (double)d.rms_eps, (int32_t)n, d.heads, (int32_t)kvh,
          (int32_t)hd, (int32_t)past, m->kv_f16,
          // the second set: every pair of the head (those beyond its share
          // have frequency 0)
          (int32_t)(L.rope_set ? 0 : rope_dims(d)), d.value_norm};
  int rc = launch(m->c, "qkrope", dim3((unsigned)(d.heads + kvh), (unsigned)n), dim3(64), &ra);
  if (rc) return rc;
  int64_t maxkeys = graph ? s->capacity : past + n;
  if (L.window > 0 && maxkeys > L.window) maxkeys = L.window;
  // a graph replays one grid for every position: splits for the longest
  return enqueue_attention(m->c, s->q, s->kc[l], s->vc[l], s->attn, s->attn_part, n, d.heads, kvh, hd, past,
                           graph ? s->pos : 0, L.window, L.sinks,
                           d.attention_scale > 0 ? d.attention_scale : 1.0 / std::sqrt((double)hd), m->kv_f16,
                           attention_splits(maxkeys));
}

// the launch arguments of deltanet.hip
struct DnConvArgs {
  float* qkv;
  const float* w;
  float* conv;
  int32_t rows, channels, kw, pad;
};
struct DnPrepArgs {
  float* qkv;
  float* beta;
  float* decay;
  float* z;
  const float* dt_bias;
  const float* neg_a;
  int32_t kh, vh, dk, dv, channels, pad;
};
struct DnConvPrepArgs {
  float* qkv;
  const float* w;
  float* conv;
  float* beta;
  float* decay;
  float* z;
  const float* dt_bias;
  const float* neg_a;
  int32_t kh, vh, dk, dv, channels, kw;
};
struct DnRuleArgs {
  const float* qkv;
  const float* beta;
  const float* decay;
  float* state;
  float* y;
  int32_t rows, stride, kh, vh, dk, dv, group, pad;
};
struct DnNormArgs {
  float* x;
  const float* w;
  const float* z;
  double eps;
  int32_t rows, cols;
};
struct GateArgs {
  const float* qg;
  float* q;
  float* g;
  int64_t n;
  int32_t hd, pad;
};
// the launch arguments of ops.hip's element-wise kernels (EltArgs) and softcap
struct EltArgs2 {
  float* x;
  const float* t;
  int64_t n;
  float alpha, limit;
};
struct SoftcapArgs {
  float* x;
  int64_t n;
  double cap;
};

// ops.hip's row_tail: a block output's norms, the experts beside it, the
// residual, the layer scalar and the next input norm in one launch
struct TailArgs {
  float* x;
  const float* t;
  const float *dn_w, *ed, *ew, *moe_w, *out_w, *scalar, *nw;
  float* h;
  double eps;
  int32_t rows, cols, k, pad;
};

static int row_tail(ihip_model* m, uint64_t x, uint64_t t, uint64_t dn_w, uint64_t ed, uint64_t ew,
                    int64_t k, uint64_t moe_w, uint64_t out_w, uint64_t scalar, uint64_t nw,
                    uint64_t h, int64_t n)
{
  const int64_t H = m->d.hidden;
  if (H > 4096 || (ed && (k < 1 || k > 16))) return fail(IHIP_E_UNSUPPORTED, "row_tail: hidden <= 4096, k <= 16");
  TailArgs a = {(float*)x, (const float*)t, (const float*)dn_w, (const float*)ed, (const float*)ew,
                (const float*)moe_w, (const float*)out_w, (const float*)scalar, (const float*)nw,
                (float*)h, m->d.rms_eps, (int32_t)n, (int32_t)H, (int32_t)k, 0};
  return launch(m->c, "row_tail", dim3((unsigned)n), dim3(1024), &a);
}

static int deltanet_block(ihip_mctx* s, int l, int64_t n, QCache* qh, bool fused = false);

// whether one row runs through layers_one: the norms fused into the GEMVs
// (hidden <= 4096), a token's experts combined in one launch (<= 8 slots)
static bool one_row_fused(const ihip_model* m)
{
  const ihip_model_desc& d = m->d;
  if (d.hidden > 4096 || m->gemma) return false;
  if (d.experts > 0) {
    const int64_t K = d.experts_used;
    if (K < 1 || K > 8 || K * d.expert_ffn * 4 > 65536) return false;
  }
  return true;
}

// TDecoderRouteTape.Take (decoder.pas:2993-3035) for the n rows the device
// just routed (their picks in ids_dev, by id, and weights in rw): each row's
// own choice compared with the tape's, then the tape's picks and weights
// written in their place for the experts that follow
static int tape_route(ihip_mctx* s, int64_t n)
{
  ihip_model* m = s->m;
  const int64_t E = m->d.experts, K = m->d.experts_used;
  if (m->tape_pos + n > m->tape_rows)
    return fail(IHIP_E_ARG, "route tape: no recorded choice left (" + std::to_string(m->tape_routes) +
                                " replayed)");
  ihip_ctx* c = m->c;
  std::vector<float> lg((size_t)(n * E));
  std::vector<int32_t> ids((size_t)(n * K));
  IHIP_CHECK(hipMemcpyDtoHAsync(lg.data(), (hipDeviceptr_t)s->route, n * E * 4, c->stream));
  IHIP_CHECK(hipMemcpyDtoHAsync(ids.data(), (hipDeviceptr_t)s->ids_dev, n * K * 4, c->stream));
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  const int32_t* tid = m->tape_ids.data() + m->tape_pos * K;
  const float* tw = m->tape_w.data() + m->tape_pos * K;
  for (int64_t r = 0; r < n; r++) {
    const int32_t* mine = ids.data() + r * K;
    bool same = true;
    for (int64_t j = 0; j < K && same; j++) {
      bool found = false;
      for (int64_t i = 0; i < K; i++) found = found || tid[r * K + i] == mine[j];
      same = found;
    }
    if (!same) {
      // the k-th highest logit of the device's choice and the highest it left out
      const float* l = lg.data() + r * E;
      double kth = INFINITY, best = -1e38;
      for (int64_t j = 0; j < K; j++) kth = std::min(kth, (double)l[mine[j]]);
      for (int64_t i = 0; i < E; i++) {
        bool picked = false;
        for (int64_t j = 0; j < K; j++) picked = picked || mine[j] == i;
        if (!picked && l[i] > best) best = l[i];
      }
      m->tape_differs++;
      m->tape_gap = std::max(m->tape_gap, kth - best);
    }
  }
  // the tape holds each row's picks in pick order (TDecoderModel.Route's
  // ranking); the device's slots hold them by id, as its own route writes
  // them and as TDecoderModel.Experts adds the experts (id order)
  std::vector<int32_t> sid((size_t)(n * K));
  std::vector<float> sw((size_t)(n * K));
  for (int64_t r = 0; r < n; r++) {
    std::vector<int64_t> ord((size_t)K);
    for (int64_t j = 0; j < K; j++) ord[j] = j;
    std::stable_sort(ord.begin(), ord.end(),
                     [&](int64_t a, int64_t b) { return tid[r * K + a] < tid[r * K + b]; });
    for (int64_t j = 0; j < K; j++) {
      sid[r * K + j] = tid[r * K + ord[j]];
      sw[r * K + j] = tw[r * K + ord[j]];
    }
  }
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->ids_dev, (void*)sid.data(), n * K * 4, c->stream));
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->rw, (void*)sw.data(), n * K * 4, c->stream));
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  m->tape_pos += n;
  m->tape_routes += n;
  return 0;
}

// CheckDeviceRoute (model.qwen3.cuda.pas:1207-1256): the router logits, the
// picks and the weights the device wrote for one row, read back after the
// route, against TDecoderModel.Route (decoder.pas:2901-2949) on the same
// logits on the host: softmax in double, the k highest (the lower id on a
// tie), NormTopK, the expert scales, then the picks sorted by id as the
// device writes them. Counts rows, rows whose ids differ and the largest
// weight difference of the others (1e30 for a NaN or infinity).
static int check_device_route(ihip_mctx* s, int l)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const int64_t E = d.experts, K = d.experts_used;
  ihip_ctx* c = m->c;
  std::vector<float> lg((size_t)E), kw((size_t)K), scale;
  std::vector<int32_t> kid((size_t)K);
  IHIP_CHECK(hipMemcpyDtoHAsync(lg.data(), (hipDeviceptr_t)s->route, E * 4, c->stream));
  IHIP_CHECK(hipMemcpyDtoHAsync(kid.data(), (hipDeviceptr_t)s->ids_dev, K * 4, c->stream));
  IHIP_CHECK(hipMemcpyDtoHAsync(kw.data(), (hipDeviceptr_t)s->rw, K * 4, c->stream));
  if (m->L[l].expert_scale) {
    scale.resize((size_t)E);
    IHIP_CHECK(hipMemcpyDtoHAsync(scale.data(), (hipDeviceptr_t)m->L[l].expert_scale, E * 4, c->stream));
  }
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  double mx = lg[0], sum = 0, picked = 0;
  for (int64_t i = 1; i < E; i++)
    if (lg[i] > mx) mx = lg[i];
  for (int64_t i = 0; i < E; i++) sum = sum + std::exp((double)lg[i] - mx);
  std::vector<int32_t> ch((size_t)K);
  std::vector<float> cw((size_t)K);
  for (int64_t j = 0; j < K; j++) {
    int64_t best = -1;
    for (int64_t i = 0; i < E; i++) {
      bool taken = false;
      for (int64_t t = 0; t < j; t++) taken = taken || ch[t] == i;
      if (!taken && (best < 0 || lg[i] > lg[best])) best = i;
    }
    ch[j] = (int32_t)best;
    cw[j] = (float)(std::exp((double)lg[best] - mx) / sum);
    picked = picked + cw[j];
  }
  if (d.norm_topk)
    for (int64_t j = 0; j < K; j++) cw[j] = (float)(cw[j] / picked);
  if (!scale.empty())
    for (int64_t j = 0; j < K; j++) cw[j] = cw[j] * scale[ch[j]];
  for (int64_t j = 1; j < K; j++) {  // by id, as the device writes them
    const int32_t id = ch[j];
    const float v = cw[j];
    int64_t t = j;
    for (; t > 0 && ch[t - 1] > id; t--) {
      ch[t] = ch[t - 1];
      cw[t] = cw[t - 1];
    }
    ch[t] = id;
    cw[t] = v;
  }
  m->route_checks++;
  for (int64_t j = 0; j < K; j++)
    if (ch[j] != kid[j]) {
      m->route_mismatches++;
      return 0;
    }
  for (int64_t j = 0; j < K; j++) {
    double dd = std::fabs((double)cw[j] - (double)kw[j]);
    if (!(dd <= 1)) dd = 1e30;
    if (dd > m->route_max_diff) m->route_max_diff = dd;
  }
  return 0;
}

// one row through the layers, x holding its embedding: every RMSNorm is
// computed by the GEMVs that read it (their staging), the residual adds by
// the GEMVs that produce them (o projection, FFN down, the experts'
// combine), so the row costs no norm or add launches. The arithmetic is that
// of layers() step for step. Leaves x = the residual (the final norm is the
// head's).
static int layers_one(ihip_mctx* s, int64_t past, bool graph)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd,
                kvw = (int64_t)d.kv_heads * hd;
  int rc = 0;
  auto normed = [&](uint64_t nw, int dt, uint64_t w, int64_t out, uint64_t bias, uint64_t y) {
    LinearCall k;
    k.x = s->x; k.rows = 1; k.in = H; k.dtype = dt; k.w = w; k.out = out; k.bias = bias;
    k.y = y; k.mode = m->mode; k.nw = nw; k.eps = d.rms_eps;
    return enqueue_linear(m->c, k);
  };
  for (int l = 0; l < d.layers; l++) {
    const DevLayer& L = m->L[l];
    if (L.mixer == IHIP_MIXER_DELTANET) {
      // the DeltaNet's projections normed in their staging, the output
      // projection adding the residual
      if ((rc = deltanet_block(s, l, 1, nullptr, true))) return rc;
      goto ffn;
    }
    // attention block (decoder.pas:2625-2702)
    {
      // q, k and v: the matrices of one weight type in one launch (a gated
      // attention's q rows: per head its query, then its gate, into qg)
      const int dts[3] = {L.qd, L.kd, L.vd};
      const uint64_t ws[3] = {L.q, L.k, L.v}, bs[3] = {L.qb, L.kb, L.vb},
                     ys[3] = {L.output_gate ? s->qg : s->q, s->k, s->v};
      const int64_t os[3] = {L.output_gate ? 2 * qw : qw, kvw, kvw};
      bool done[3] = {false, false, false};
      // two types with a kernel for the pair (Q4_K_M: q, k Q4_K and v Q6_K)
      int t2 = 0;
      for (int j = 1; j < 3; j++)
        if (dts[j] != dts[0]) t2 = t2 ? (dts[j] == t2 ? t2 : -1) : dts[j];
      if (t2 > 0 && gemv_pair(m->c, dts[0], t2, m->mode, H)) {
        LinearCall k;
        k.x = s->x; k.rows = 1; k.in = H; k.dtype = dts[0]; k.dtype2 = t2; k.mode = m->mode;
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
        k.x = s->x; k.rows = 1; k.in = H; k.dtype = dts[i]; k.mode = m->mode;
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
      if (L.output_gate) {
        GateArgs ga = {(const float*)s->qg, (float*)s->q, (float*)s->gq, qw, (int32_t)hd, 0};
        if ((rc = launch(m->c, "split_gate", dim3((unsigned)((qw + 255) / 256)), dim3(256), &ga))) return rc;
      }
    }
    if ((hd == 64 || hd == 128) && rope_dims(d) == hd) {
      // head norms, RoPE, cache store and the ranges in one launch, then the merge
      AttnOne o;
      o.q = s->q; o.k = s->k; o.v = s->v; o.qn = L.qn; o.kn = L.kn; o.cs = L.no_rope ? 0 : s->cs;
      o.kc = s->kc[l]; o.vc = s->vc[l]; o.y = s->attn; o.sinks = L.sinks; o.pastp = graph ? s->pos : 0;
      o.part = s->attn_part; o.scale = 1.0 / std::sqrt((double)hd);
      o.eps = d.rms_eps; o.heads = d.heads; o.kvh = d.kv_heads; o.hd = hd; o.past = past;
      o.window = L.window; o.f16 = m->kv_f16;
      if (d.heads <= 256) o.done = s->done;  // the merge in the last range block of a head
      int64_t maxkeys = graph ? s->capacity : past + 1;
      if (L.window > 0 && maxkeys > L.window) maxkeys = L.window;
      o.splits = attention_splits(maxkeys);
      if ((rc = enqueue_attention_one(m->c, o))) return rc;
    } else if ((rc = rope_attn(s, l, 1, past, graph))) {
      return rc;
    }
    if (L.output_gate) {
      // GateBySigmoid (decoder.pas:2594-2610) before the output projection
      GateArgs ga = {nullptr, (float*)s->attn, (float*)s->gq, qw, (int32_t)hd, 0};
      if ((rc = launch(m->c, "gate_sigmoid", dim3((unsigned)((qw + 255) / 256)), dim3(256), &ga))) return rc;
    }
    {
      LinearCall k;
      k.x = s->attn; k.rows = 1; k.in = qw; k.dtype = L.od; k.w = L.o; k.out = H; k.bias = L.ob;
      k.y = s->x; k.res = s->x; k.mode = m->mode;
      if ((rc = enqueue_linear(m->c, k))) return rc;
    }
  ffn:
    if (!L.moe) {
      // DenseFfn (decoder.pas:2866-2878): gate, up and SwiGLU in one pass
      const int64_t F = d.ffn;
      if (L.gd != L.ud) return fail(IHIP_E_ARG, "model: gate and up of one type");
      LinearCall k;
      k.x = s->x; k.rows = 1; k.in = H; k.dtype = L.gd; k.w = L.gate; k.out = F;
      k.y = s->gate; k.mode = m->mode; k.w2 = L.up; k.alpha = d.swiglu_alpha;
      k.limit = d.swiglu_limit; k.nw = L.post_norm; k.eps = d.rms_eps;
      if ((rc = enqueue_linear(m->c, k))) return rc;
      LinearCall dn;
      dn.x = s->gate; dn.rows = 1; dn.in = F; dn.dtype = L.dd; dn.w = L.down; dn.out = H;
      dn.y = s->x; dn.res = s->x; dn.mode = m->mode;
      if ((rc = enqueue_linear(m->c, dn))) return rc;
      continue;
    }
    // MoeBlock (decoder.pas:3037-3053), the experts chosen on the device
    const int64_t E = d.experts, K = d.experts_used, FI = d.expert_ffn;
    // the router's launch also writes the normed row quantized for the
    // experts' gate/up (float router weights, the Q8 arithmetic): the same
    // rmsnorm and quantization as the experts' own staging would form, once
    const int xk = q8_kind(L.egd);
    const bool xq_pass = (m->mode & 1) == IHIP_MODE_Q8 && xk >= 0 &&
                         (L.rd == DT_F32 || L.rd == DT_BF16 || L.rd == DT_F16) && H <= 4096 &&
                         (xk == 0 || H % 256 == 0);
    const uint64_t xqr = xk == 1 ? s->xqk : s->xq0;
    {
      LinearCall k;
      k.x = s->x; k.rows = 1; k.in = H; k.dtype = L.rd; k.w = L.router; k.out = E; k.bias = L.router_b;
      k.y = s->route; k.mode = m->mode; k.nw = L.post_norm; k.eps = d.rms_eps;
      if (xq_pass) {
        k.xq_out = xqr;
        k.xq_k8 = xk == 1;
      }
      if ((rc = enqueue_linear(m->c, k))) return rc;
    }
    // the route (TDecoderModel.Route) inside the gate/up launch: each block
    // ranks the logits for its slot's expert, one writes the picks and
    // weights for the down launch (up to 256 experts); else its own launch
    const bool taped = m->tape_rows > 0 && !m->c->capturing;
    const bool self_route = E <= 256 && K <= E && K <= 8 && !taped;
    if (!self_route) {
      struct {
        const float* logits;
        int* ids;
        float* w;
        int32_t experts, k, norm, rows;
        const float* scale;
      } ra = {(const float*)s->route, (int*)s->ids_dev, (float*)s->rw, (int32_t)E, (int32_t)K,
              d.norm_topk, 1};
      if ((rc = launch(m->c, "route", dim3(1), dim3(256), &ra))) return rc;
      if (taped && (rc = tape_route(s, 1))) return rc;
    }
    LinearCall k;
    k.x = s->x; k.rows = K; k.in = H; k.dtype = L.egd; k.w = L.eg; k.out = FI;
    k.y = s->gate; k.mode = m->mode; k.ids = s->ids_dev; k.stride = L.eg_stride; k.x_per_slot = 0;
    k.nexp = (int)E; k.bias = L.egb; k.w2 = L.eu; k.bias2 = L.eub; k.alpha = d.swiglu_alpha;
    k.limit = d.swiglu_limit; k.nw = L.post_norm; k.eps = d.rms_eps;
    if (xq_pass) {
      // the router's quantized normed row (the norm is not formed again)
      k.x = xqr; k.nw = 0; k.mode = m->mode | IHIP_MODE_XQ;
    }
    if (self_route) {
      k.rl = s->route; k.rw = s->rw; k.rexp = (int)E; k.rk = (int)K; k.rnorm = d.norm_topk;
    }
    if ((rc = enqueue_linear(m->c, k))) return rc;
    if (m->check_route && !m->c->capturing && (rc = check_device_route(s, l))) return rc;
    LinearCall dn;
    dn.x = s->gate; dn.rows = K; dn.in = FI; dn.dtype = L.edd; dn.w = L.ed; dn.out = H;
    dn.y = s->x; dn.res = s->x; dn.cw = s->rw; dn.mode = m->mode; dn.ids = s->ids_dev;
    dn.stride = L.ed_stride; dn.x_per_slot = 1; dn.nexp = (int)E; dn.bias = L.edb;
    if ((rc = enqueue_linear(m->c, dn))) return rc;
  }
  return 0;
}


// DeltaNetBlock (decoder.pas:2704-2753) of layer l over n rows, h holding
// their input norm: the four projections, the convolution and DeltaPrep, the
// delta rule on the layer's state, the gated RMSNorm, the output projection
// into tmp
static int deltanet_block(ihip_mctx* s, int l, int64_t n, QCache* qh, bool fused)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const DevLayer& L = m->L[l];
  const int64_t H = d.hidden, kh = d.lin_key_heads, vh = d.lin_value_heads, dk = d.lin_key_dim,
                dv = d.lin_value_dim, vd = vh * dv, cd = 2 * kh * dk + vd;
  int rc;
  uint64_t decay = s->decay;
  if (fused) {
    // one row, x the residual: every projection norms it in its staging; the
    // q/k/v channels, z and beta|alpha (one matrix when their types match,
    // decay then after beta) in one launch of one weight type
    LinearCall k;
    k.x = s->x; k.rows = 1; k.in = H; k.mode = m->mode; k.nw = L.input_norm; k.eps = d.rms_eps;
    auto seg = [&](uint64_t w, int64_t out, uint64_t y) {
      k.wseg[k.nseg] = w; k.oseg[k.nseg] = out; k.yseg[k.nseg] = y; k.bseg[k.nseg] = 0; k.nseg++;
    };
    if (L.lba && L.lqkvd == L.lzd && L.lzd == L.lbad) {
      k.dtype = L.lqkvd;
      seg(L.lqkv, cd, s->qkv);
      seg(L.lz, vd, s->z);
      seg(L.lba, 2 * vh, s->beta);
      k.w = k.wseg[0]; k.y = k.yseg[0]; k.out = k.oseg[0];
      if ((rc = enqueue_linear(m->c, k))) return rc;
      decay = s->beta + (uint64_t)vh * 4;
    } else {
      const int dts[4] = {L.lqkvd, L.lzd, L.lbd, L.lad};
      const uint64_t ws[4] = {L.lqkv, L.lz, L.lb, L.la}, ys[4] = {s->qkv, s->z, s->beta, s->decay};
      const int64_t os[4] = {cd, vd, vh, vh};
      for (int i = 0; i < 4; i++) {
        LinearCall one;
        one.x = s->x; one.rows = 1; one.in = H; one.dtype = dts[i]; one.w = ws[i]; one.out = os[i];
        one.y = ys[i]; one.mode = m->mode; one.nw = L.input_norm; one.eps = d.rms_eps;
        if ((rc = enqueue_linear(m->c, one))) return rc;
      }
    }
  } else if ((rc = lin(s, s->h, qh, n, H, L.lqkvd, L.lqkv, cd, 0, s->qkv)) ||
             (rc = lin(s, s->h, qh, n, H, L.lzd, L.lz, vd, 0, s->z)) ||
             (rc = lin(s, s->h, qh, n, H, L.lbd, L.lb, vh, 0, s->beta)) ||
             (rc = lin(s, s->h, qh, n, H, L.lad, L.la, vh, 0, s->decay))) {
    return rc;
  }
  if (n == 1 && dv <= 256) {
    // one row: the convolution and DeltaPrep of each item in one launch (a
    // wave holds an item's channels, up to 256)
    DnConvPrepArgs cp = {(float*)s->qkv, (const float*)L.lconv, (float*)s->conv[l], (float*)s->beta, (float*)decay,
                         (float*)s->z, (const float*)L.ldt, (const float*)L.lnega, (int32_t)kh, (int32_t)vh,
                         (int32_t)dk, (int32_t)dv, (int32_t)cd, d.lin_conv};
    if ((rc = launch(m->c, "dn_convprep1", dim3((unsigned)(2 * kh + vh)), dim3(64), &cp))) return rc;
  } else {
    DnConvArgs ca = {(float*)s->qkv, (const float*)L.lconv, (float*)s->conv[l], (int32_t)n, (int32_t)cd,
                     d.lin_conv, 0};
    if ((rc = launch(m->c, "dn_conv", dim3((unsigned)((cd + 255) / 256)), dim3(256), &ca))) return rc;
    DnPrepArgs pa = {(float*)s->qkv, (float*)s->beta, (float*)decay, (float*)s->z, (const float*)L.ldt,
                     (const float*)L.lnega, (int32_t)kh, (int32_t)vh, (int32_t)dk, (int32_t)dv, (int32_t)cd, 0};
    if ((rc = launch(m->c, "dn_prep", dim3((unsigned)(2 * kh + vh), (unsigned)n), dim3(64), &pa))) return rc;
  }
  // LinGroup (decoder.pas:2457-2463)
  const int32_t group = d.lin_tiled ? 1 : (int32_t)(vh / kh);
  DnRuleArgs ra = {(const float*)s->qkv, (const float*)s->beta, (const float*)decay, (float*)s->state[l],
                   (float*)s->core, (int32_t)n, (int32_t)cd, (int32_t)kh, (int32_t)vh, (int32_t)dk,
                   (int32_t)dv, group, 0};
  if ((rc = launch(m->c, "dn_rule", dim3((unsigned)vh, (unsigned)((dv + 3) / 4)), dim3(256), &ra))) return rc;
  DnNormArgs na = {(float*)s->core, (const float*)L.lnorm, (const float*)s->z, (double)d.rms_eps,
                   (int32_t)(n * vh), (int32_t)dv};
  if ((rc = launch(m->c, "dn_gatenorm", dim3((unsigned)((n * vh + 3) / 4)), dim3(256), &na))) return rc;
  if (fused) {
    // the output projection adds the residual
    LinearCall k;
    k.x = s->core; k.rows = 1; k.in = vd; k.dtype = L.loutd; k.w = L.lout; k.out = H;
    k.y = s->x; k.res = s->x; k.mode = m->mode;
    return enqueue_linear(m->c, k);
  }
  QCache qc{s->xq0, s->xqk};
  return lin(s, s->core, n == 1 ? nullptr : &qc, n, vd, L.loutd, L.lout, H, 0, s->tmp);
}

// a new sequence: the convolution sees zeros before it, the states are 0
// (DeltaNetBlock, decoder.pas:2723-2729); outside any capture
static int reset_states(ihip_mctx* s)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const int64_t cd = 2 * (int64_t)d.lin_key_heads * d.lin_key_dim + (int64_t)d.lin_value_heads * d.lin_value_dim;
  for (int l = 0; l < d.layers; l++) {
    if (!s->conv[l]) continue;
    IHIP_CHECK(hipMemsetAsync((void*)s->conv[l], 0, (size_t)cd * std::max(d.lin_conv - 1, 1) * 4,
                              m->c->stream));
    IHIP_CHECK(hipMemsetAsync((void*)s->state[l], 0,
                              (size_t)d.lin_value_heads * d.lin_value_dim * d.lin_key_dim * 4, m->c->stream));
  }
  return 0;
}

// the layers of one chunk of n rows at positions past.., x holding the
// embeddings; leaves h = the final norm of x. graph: the position is read
// from s->pos (decode step under capture)
static int layers(ihip_mctx* s, int64_t n, int64_t past, bool graph)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden;
  // one row (decode): every GEMV quantizes its activation row in registers;
  // a chunk: the rows are quantized once per activation buffer
  const bool one = n == 1;
  if (one && one_row_fused(m)) return layers_one(s, past, graph);
  // the gate/up activation fused into a one-row GEMV: SwiGLU, or GeGLU
  // (the kernels' limit < 0)
  const bool glu_fused = one && (d.activation == IHIP_ACT_SILU || d.activation == IHIP_ACT_GELU_TANH);
  const float glu_limit = d.activation == IHIP_ACT_GELU_TANH ? -1.0f : d.swiglu_limit;
  // TDecoderModel.Activate (decoder.pas:2857-2863): SwiGLU or GeGLU in place
  auto activate = [&](uint64_t gate, uint64_t up, int64_t count) {
    if (d.activation == IHIP_ACT_GELU_TANH) {
      EltArgs2 ea = {(float*)gate, (const float*)up, count, 0.f, 0.f};
      return launch(m->c, "geglu", dim3((unsigned)((count + 255) / 256)), dim3(256), &ea);
    }
    return ihip_enqueue_swiglu(m->c, gate, up, count, d.swiglu_alpha, d.swiglu_limit);
  };
  auto norm = [&](uint64_t x, uint64_t w, uint64_t y) { return ihip_enqueue_rmsnorm(m->c, x, w, y, n, H, d.rms_eps); };
  int rc = norm(s->x, m->L[0].input_norm, s->h);
  if (rc) return rc;
  // a test's capture of the residual rows after layer dbg_layer (a chunk)
  auto capture = [&](int l) -> int {
    if (!m->dbg_host || (m->dbg_layer >= 0 && l != m->dbg_layer)) return 0;
    float* dst = m->dbg_host + (m->dbg_layer < 0 ? (size_t)l * n * H : 0);
    IHIP_CHECK(hipMemcpyDtoHAsync(dst, (hipDeviceptr_t)s->x, (size_t)n * H * 4, m->c->stream));
    IHIP_CHECK(hipStreamSynchronize(m->c->stream));
    return 0;
  };
  for (int l = 0; l < d.layers; l++) {
    if (l > 0 && (rc = capture(l - 1))) return rc;
    const DevLayer& L = m->L[l];
    const int64_t hd = L.hd, qw = (int64_t)d.heads * hd, kvw = L.kvh * hd;
    QCache qh{s->xq0, s->xqk};
    QCache* qhp = one ? nullptr : &qh;
    if (L.mixer == IHIP_MIXER_DELTANET) {
      if ((rc = deltanet_block(s, l, n, qhp))) return rc;
    } else {
      // attention block (decoder.pas:2625-2702)
      if (L.output_gate) {
        // per head the query, then its gate: apart into q and gq
        if ((rc = lin(s, s->h, qhp, n, H, L.qd, L.q, 2 * qw, 0, s->qg))) return rc;
        GateArgs ga = {(const float*)s->qg, (float*)s->q, (float*)s->gq, n * qw, (int32_t)hd, 0};
        if ((rc = launch(m->c, "split_gate", dim3((unsigned)((n * qw + 255) / 256)), dim3(256), &ga)))
          return rc;
      } else if (one && L.qd == L.kd && (L.k_is_v || L.vd == L.qd)) {
        // one row: q, k and v (k alone when V is K) as the matrices of one launch
        LinearCall k;
        k.x = s->h; k.rows = 1; k.in = H; k.dtype = L.qd; k.mode = m->mode;
        k.nseg = L.k_is_v ? 2 : 3;
        k.wseg[0] = L.q; k.wseg[1] = L.k; k.wseg[2] = L.v;
        k.bseg[0] = L.qb; k.bseg[1] = L.kb; k.bseg[2] = L.vb;
        k.yseg[0] = s->q; k.yseg[1] = s->k; k.yseg[2] = s->v;
        k.oseg[0] = qw; k.oseg[1] = kvw; k.oseg[2] = kvw;
        k.w = L.q; k.out = qw; k.y = s->q; k.bias = L.qb;
        if ((rc = enqueue_linear(m->c, k))) return rc;
        goto attend;
      } else if ((rc = lin(s, s->h, qhp, n, H, L.qd, L.q, qw, L.qb, s->q))) {
        return rc;
      }
      if ((rc = lin(s, s->h, qhp, n, H, L.kd, L.k, kvw, L.kb, s->k))) return rc;
      if (!L.k_is_v && (rc = lin(s, s->h, qhp, n, H, L.vd, L.v, kvw, L.vb, s->v))) return rc;
    attend:
      if ((rc = rope_attn(s, l, n, past, graph))) return rc;
      if (L.output_gate) {
        // GateBySigmoid (decoder.pas:2594-2610) before the output projection
        GateArgs ga = {nullptr, (float*)s->attn, (float*)s->gq, n * qw, (int32_t)hd, 0};
        if ((rc = launch(m->c, "gate_sigmoid", dim3((unsigned)((n * qw + 255) / 256)), dim3(256), &ga)))
          return rc;
      }
      QCache qa{s->xq0, s->xqk};
      if ((rc = lin(s, s->attn, one ? nullptr : &qa, n, qw, L.od, L.o, H, L.ob, s->tmp))) return rc;
    }
    // residual, then the pre-FFN norm; Gemma norms the attention output
    // before the residual
    if (L.attn_out_norm && L.mixer != IHIP_MIXER_DELTANET && H <= 4096)
      rc = row_tail(m, s->x, s->tmp, 0, 0, 0, 0, 0, L.attn_out_norm, 0, L.post_norm, s->h, n);
    else if (L.attn_out_norm && L.mixer != IHIP_MIXER_DELTANET && (rc = norm(s->tmp, L.attn_out_norm, s->tmp)))
      return rc;
    else
      rc = ihip_enqueue_addnorm(m->c, s->x, s->tmp, L.post_norm, s->h, n, H, d.rms_eps);
    if (rc) return rc;
    QCache qf{s->xq0, s->xqk};
    QCache* qfp = one ? nullptr : &qf;
    bool moe_out = false;  // the FFN output is the expert rows (added by the next norm)
    if (L.moe != IHIP_FFN_MOE) {
      // DenseFfn (decoder.pas:2866-2878)
      const int64_t F = d.ffn;
      if (glu_fused) {
        // gate, up and SwiGLU in one pass
        LinearCall k;
        k.x = s->h; k.rows = 1; k.in = H; k.dtype = L.gd; k.w = L.gate; k.out = F;
        k.y = s->gate; k.mode = m->mode; k.w2 = L.up; k.alpha = d.swiglu_alpha;
        k.limit = glu_limit;
        if (L.gd != L.ud) return fail(IHIP_E_ARG, "model: gate and up of one type");
        if ((rc = enqueue_linear(m->c, k))) return rc;
      } else {
        if ((rc = lin(s, s->h, qfp, n, H, L.gd, L.gate, F, 0, s->gate))) return rc;
        if ((rc = lin(s, s->h, qfp, n, H, L.ud, L.up, F, 0, s->up))) return rc;
        if ((rc = activate(s->gate, s->up, n * F))) return rc;
      }
      QCache qg{s->xqf, s->xqf};
      if ((rc = lin(s, s->gate, one ? nullptr : &qg, n, F, L.dd, L.down, H, 0, s->tmp))) return rc;
    }
    if (L.moe != IHIP_FFN_DENSE) {
      // MoeBlock (decoder.pas:3037-3053) with the experts chosen on the
      // device (model.qwen3.cuda.pas:1152-1205); DenseMoeBlock (:3057-3091):
      // the dense output normed, the router on the residual's own norm, the
      // experts on another, their sum normed
      const bool beside = L.moe == IHIP_FFN_DENSE_MOE;
      const int64_t E = d.experts, K = d.experts_used, FI = d.expert_ffn;
      QCache qr{s->xq0, s->xqk};
      QCache* qx = qfp;
      // the tail: the dense output's norm waits for row_tail below when it
      // fits (nothing reads it before)
      const bool tailed = beside && H <= 4096 && K <= 16;
      // one row beside the dense block: the router and the experts norm the
      // residual in their staging (router_norm, moe_in_norm)
      const bool staged = beside && glu_fused;
      if (beside) {
        if ((!tailed && (rc = norm(s->tmp, L.dense_out_norm, s->tmp))) ||
            (!staged && (rc = norm(s->x, L.router_norm, s->h))))
          return rc;
        qx = one ? nullptr : &qr;
      }
      if (staged) {
        LinearCall k;
        k.x = s->x; k.rows = 1; k.in = H; k.dtype = L.rd; k.w = L.router; k.out = E; k.bias = L.router_b;
        k.y = s->route; k.mode = m->mode; k.nw = L.router_norm; k.eps = d.rms_eps;
        if ((rc = enqueue_linear(m->c, k))) return rc;
      } else if ((rc = lin(s, s->h, qx, n, H, L.rd, L.router, E, L.router_b, s->route))) {
        return rc;
      }
      struct {
        const float* logits;
        int* ids;
        float* w;
        int32_t experts, k, norm, rows;
        const float* scale;
      } ra = {(const float*)s->route, (int*)s->ids_dev, (float*)s->rw, (int32_t)E, (int32_t)K,
              d.norm_topk, (int32_t)n, (const float*)L.expert_scale};
      // one row beside the dense block: the route formed in the experts'
      // gate/up launch (route_wave, the expert scales applied as route does)
      const bool taped = m->tape_rows > 0 && !m->c->capturing;
      const bool self_route = staged && E <= 256 && K <= E && K <= 8 && !taped;
      if (!self_route && (rc = launch(m->c, "route", dim3((unsigned)n), dim3(256), &ra))) return rc;
      if (taped && (rc = tape_route(s, n))) return rc;
      QCache qe{s->xq0, s->xqk};
      if (beside && !staged) {
        if ((rc = norm(s->x, L.moe_in_norm, s->h))) return rc;
        qf = qe;
      }
      if (glu_fused) {
        // the token's K experts: gate, up and SwiGLU in one pass per slot,
        // then down per slot; the weighted sum goes into the next norm
        LinearCall k;
        k.x = staged ? s->x : s->h; k.rows = K; k.in = H; k.dtype = L.egd; k.w = L.eg; k.out = FI;
        k.y = s->gate; k.mode = m->mode; k.ids = s->ids_dev; k.stride = L.eg_stride; k.x_per_slot = 0;
        k.nexp = (int)E; k.bias = L.egb; k.w2 = L.eu; k.bias2 = L.eub; k.alpha = d.swiglu_alpha;
        k.limit = glu_limit;
        if (staged) {
          k.nw = L.moe_in_norm;
          k.eps = d.rms_eps;
        }
        if (self_route) {
          k.rl = s->route; k.rw = s->rw; k.rexp = (int)E; k.rk = (int)K; k.rnorm = d.norm_topk;
          k.rscale = L.expert_scale;
        }
        if ((rc = enqueue_linear(m->c, k))) return rc;
        if (n == 1 && m->check_route && !m->c->capturing && (rc = check_device_route(s, l))) return rc;
        LinearCall dn;
        dn.x = s->gate; dn.rows = K; dn.in = FI; dn.dtype = L.edd; dn.w = L.ed; dn.out = H;
        dn.y = s->eout; dn.mode = m->mode; dn.ids = s->ids_dev; dn.stride = L.ed_stride;
        dn.x_per_slot = 1; dn.nexp = (int)E; dn.bias = L.edb;
        if (tailed && K <= 8 && K * FI * 4 <= 65536) {
          // the slots' weighted sum in slot order in the same launch
          // (moecombine's arithmetic), into the experts' row of the tail
          dn.y = s->moe; dn.cw = s->rw;
        }
        if ((rc = enqueue_linear(m->c, dn))) return rc;
      } else {
        struct {
          const int* ids;
          int* perm;
          void* items;
          int32_t slots, experts, max_items, chunk;
        } pa = {(const int*)s->ids_dev, (int*)s->perm, (void*)s->items, (int32_t)(n * K), (int32_t)E,
                (int32_t)((n * K + m->item_rows - 1) / m->item_rows + E), m->item_rows};
        if ((rc = launch(m->c, "moe_plan", dim3(1), dim3(256), &pa))) return rc;
        // gate and up: slot s = row s / K, expert ids[s], grouped by expert
        bool q0 = false;
        if (m->mode == IHIP_MODE_Q8 && q8_kind(L.egd) >= 0) {
          bool& hv = q8_kind(L.egd) ? qf.havek : qf.have0;
          uint64_t buf = q8_kind(L.egd) ? qf.bufk : qf.buf0;
          if (!hv) {
            if ((rc = enqueue_quantize(m->c, s->h, n, H, q8_kind(L.egd), buf))) return rc;
            hv = true;
          }
          q0 = true;
        }
        uint64_t xqg = q8_kind(L.egd) == 1 ? qf.bufk : qf.buf0;
        if ((rc = lin_ids(s, s->h, xqg, n, H, L.egd, L.eg, L.eg_stride, FI, s->ids_dev, n * K, (int)K,
                          L.egb, s->gate, q0)))
          return rc;
        bool qu = q0 && q8_kind(L.eud) == q8_kind(L.egd);
        uint64_t xqu = q8_kind(L.eud) == 1 ? qf.bufk : qf.buf0;
        if ((rc = lin_ids(s, s->h, xqu, n, H, L.eud, L.eu, L.eg_stride, FI, s->ids_dev, n * K, (int)K,
                          L.eub, s->up, qu)))
          return rc;
        if ((rc = activate(s->gate, s->up, n * K * FI))) return rc;
        if ((rc = lin_ids(s, s->gate, s->xqf, n * K, FI, L.edd, L.ed, L.ed_stride, H, s->ids_dev,
                          n * K, 1, L.edb, s->eout, false)))
          return rc;
      }
      if (tailed) {
        // the experts' sum, its norm and the dense output's: row_tail below
      } else if (beside) {
        // the experts' sum in slot (= id) order, normed, added to the dense
        // output, normed again (below, as the FFN output norm)
        struct {
          const float* d;
          const float* w;
          float* y;
          int32_t k, n, rows, pad;
        } ca = {(const float*)s->eout, (const float*)s->rw, (float*)s->moe, (int32_t)K, (int32_t)H, (int32_t)n, 0};
        if ((rc = launch(m->c, "moecombine", dim3((unsigned)((H + 255) / 256), (unsigned)n), dim3(256), &ca)) ||
            (rc = norm(s->moe, L.moe_out_norm, s->moe)) || (rc = ihip_enqueue_add(m->c, s->tmp, s->moe, n * H)))
          return rc;
      } else {
        moe_out = true;
      }
    }
    // residual, then the next layer's input norm (or the final norm); Gemma
    // norms the feed-forward output before the residual and scales the whole
    // state by the layer's scalar between the two
    uint64_t nw = l + 1 < d.layers ? m->L[l + 1].input_norm : m->final_norm;
    const bool beside = L.moe == IHIP_FFN_DENSE_MOE;
    if (!moe_out && H <= 4096 && d.experts_used <= 16 && (beside || L.ffn_out_norm || L.scalar)) {
      // one row: the expert rows were combined by their down launch
      const bool combined = beside && glu_fused && d.experts_used <= 8 &&
                            d.experts_used * d.expert_ffn * 4 <= 65536;
      rc = row_tail(m, s->x, s->tmp, beside ? L.dense_out_norm : 0,
                    beside ? (combined ? s->moe : s->eout) : 0, beside && !combined ? s->rw : 0,
                    combined ? 1 : d.experts_used, beside ? L.moe_out_norm : 0, L.ffn_out_norm,
                    L.scalar, nw, s->h, n);
      if (rc) return rc;
      continue;
    }
    if (L.ffn_out_norm && (rc = norm(s->tmp, L.ffn_out_norm, s->tmp))) return rc;
    if (L.scalar) {
      if (moe_out) return fail(IHIP_E_ARG, "model: a layer scalar after experts alone");
      EltArgs2 sa = {(float*)s->x, (const float*)L.scalar, n * H, 0.f, 0.f};
      if ((rc = ihip_enqueue_add(m->c, s->x, s->tmp, n * H)) ||
          (rc = launch(m->c, "mul_scalar", dim3((unsigned)((n * H + 255) / 256)), dim3(256), &sa)))
        return rc;
      rc = norm(s->x, nw, s->h);
    } else if (moe_out) {
      rc = enqueue_addnorm_moe(m->c, s->x, s->eout, s->rw, d.experts_used, nw, s->h, n, H, d.rms_eps);
    } else {
      rc = ihip_enqueue_addnorm(m->c, s->x, s->tmp, nw, s->h, n, H, d.rms_eps);
    }
    if (rc) return rc;
  }
  if ((rc = capture(d.layers - 1))) return rc;
  return 0;
}

static int head(ihip_mctx* s, int64_t n, bool all, uint64_t y)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  QCache qh{s->xq0, s->xqk};
  if (n == 1 && one_row_fused(m)) {
    // layers_one left the residual: the final norm is staged by the head
    LinearCall k;
    k.x = s->x; k.rows = 1; k.in = d.hidden; k.dtype = m->head_dt; k.w = m->head;
    k.out = d.vocab; k.y = y; k.mode = m->mode; k.nw = m->final_norm; k.eps = d.rms_eps;
    return enqueue_linear(m->c, k);
  }
  if (all) return lin(s, s->h, &qh, n, d.hidden, m->head_dt, m->head, d.vocab, 0, y);
  return lin(s, s->h + (uint64_t)(n - 1) * d.hidden * 4, nullptr, 1, d.hidden, m->head_dt,
             m->head, d.vocab, 0, y);
}

// ---- restore points of a recurrent state (TDecoderContext,
// decoder.pas:996-1230)

static int dalloc_ctx(ihip_mctx* s, uint64_t bytes, uint64_t& p);
static void free_owned(ihip_mctx* s, uint64_t& p);

static bool ckpt_on(const ihip_mctx* s) { return s->m->recurrent && s->ckpt_id >= 0 && s->ckpt_max > 0; }

static int64_t find_ckpt(const ihip_mctx* s, int64_t length)
{
  for (size_t i = 0; i < s->ckpts.size(); i++)
    if (s->ckpts[i].first == length) return (int64_t)i;
  return -1;
}

// SaveStates / LoadStates: every DeltaNet layer's conv and state to or from
// a slot (device copies on the stream)
static int copy_states(ihip_mctx* s, int slot, bool save)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  const int64_t vd = (int64_t)d.lin_value_heads * d.lin_value_dim, cd = 2 * (int64_t)d.lin_key_heads * d.lin_key_dim + vd;
  const uint64_t cb = (uint64_t)cd * std::max(d.lin_conv - 1, 1) * 4, sb = (uint64_t)vd * d.lin_key_dim * 4;
  if (save && slot >= (int)s->slot_conv.size()) {
    s->slot_conv.resize(slot + 1, std::vector<uint64_t>(d.layers, 0));
    s->slot_state.resize(slot + 1, std::vector<uint64_t>(d.layers, 0));
  }
  for (int l = 0; l < d.layers; l++) {
    if (!s->conv[l]) continue;
    uint64_t& pc = s->slot_conv[slot][l];
    uint64_t& ps = s->slot_state[slot][l];
    int rc;
    if (!pc && ((rc = dalloc_ctx(s, cb, pc)) || (rc = dalloc_ctx(s, sb, ps)))) return rc;
    const uint64_t dc = save ? pc : s->conv[l], sc = save ? s->conv[l] : pc;
    const uint64_t ds = save ? ps : s->state[l], ss = save ? s->state[l] : ps;
    IHIP_CHECK(hipMemcpyDtoDAsync((hipDeviceptr_t)dc, (hipDeviceptr_t)sc, cb, m->c->stream));
    IHIP_CHECK(hipMemcpyDtoDAsync((hipDeviceptr_t)ds, (hipDeviceptr_t)ss, sb, m->c->stream));
  }
  return 0;
}

// SaveCheckpoint (decoder.pas:1049-1081): the states of the cached rows, when
// they are whole, aligned and new; the oldest goes when the count is full
static int save_checkpoint(ihip_mctx* s)
{
  if (s->ckpt_max <= 0 || s->length == 0 || !s->state_ok || !s->aligned || find_ckpt(s, s->length) >= 0)
    return 0;
  int slot = -1;
  if ((int64_t)s->ckpts.size() >= s->ckpt_max) {
    slot = s->ckpts.front().second;
    s->ckpts.erase(s->ckpts.begin());
  } else {
    // the lowest slot no restore point uses
    for (int k = 0; slot < 0; k++) {
      bool used = false;
      for (auto& c : s->ckpts) used = used || c.second == k;
      if (!used) slot = k;
    }
  }
  int rc = copy_states(s, slot, true);
  if (rc) return rc;
  s->ckpts.emplace_back(s->length, slot);
  return 0;
}

// a forward part starting at token id (-1: an embedding row), the first of
// its call or the start of a chunk: CheckPart (decoder.pas:1083-1102) and the
// restore point before a CheckpointId token (ForwardRows, :3230-3237)
static int part_start(ihip_mctx* s, int32_t id, bool first)
{
  if (!s->m->recurrent) return 0;
  if (s->length > 0 && !s->state_ok)
    return fail(IHIP_E_ARG, "forward: the recurrent state is undone by an earlier failure - reset it, or "
                            "truncate it to a restore point");
  if (ckpt_on(s) && s->length > 0 && id == s->ckpt_id) {
    int rc = save_checkpoint(s);
    if (rc) return rc;
  } else if (first && s->length > 0 && s->ckpt_id >= 0) {
    s->aligned = false;
  }
  s->state_ok = false;
  return 0;
}

// Restorable (decoder.pas:1180-1211): the device cache keeps every row, so
// only a recurrent state limits the lengths a context can go back to
static bool restorable(const ihip_mctx* s, int64_t length)
{
  if (length < 0 || length > s->length) return false;
  if (length == 0) return true;
  if (s->m->recurrent && (length != s->length || !s->state_ok) && find_ckpt(s, length) < 0) return false;
  return true;
}

// Truncate (decoder.pas:996-1017)
static int truncate_to(ihip_mctx* s, int64_t length)
{
  if (!restorable(s, length))
    return fail(IHIP_E_ARG, "truncate(" + std::to_string(length) + ") of " + std::to_string(s->length) +
                                " tokens: a recurrent state cannot go back there");
  if (length == 0) {
    s->length = 0;
    s->ckpts.clear();
    s->aligned = true;
    s->state_ok = true;
    return 0;
  }
  if (s->m->recurrent && (length != s->length || !s->state_ok)) {
    int rc = copy_states(s, s->ckpts[find_ckpt(s, length)].second, false);
    if (rc) return rc;
    s->state_ok = true;
    s->aligned = true;
  }
  s->length = length;
  while (!s->ckpts.empty() && s->ckpts.back().first > length) s->ckpts.pop_back();
  return 0;
}

// Gemma: the embeddings of ids times the embedding scale (ForwardPart,
// decoder.pas:3305-3309)
static int embed_scale(ihip_mctx* s, int64_t n)
{
  ihip_model* m = s->m;
  if (!(m->d.embed_scale > 0)) return 0;
  EltArgs2 a = {(float*)s->x, nullptr, n * m->d.hidden, m->d.embed_scale, 0.f};
  return launch(m->c, "mul_scalar", dim3((unsigned)((n * m->d.hidden + 255) / 256)), dim3(256), &a);
}

// Gemma: the logits soft-capped (InferSoftcap, decoder.pas:3360-3368), before
// any pick
static int softcap(ihip_mctx* s, int64_t rows, uint64_t logits)
{
  ihip_model* m = s->m;
  if (!(m->d.logit_softcap > 0)) return 0;
  SoftcapArgs a = {(float*)logits, rows * m->d.vocab, m->d.logit_softcap};
  return launch(m->c, "softcap", dim3((unsigned)((a.n + 255) / 256)), dim3(256), &a);
}

// one chunk: ids (or embedding rows) and cos/sin uploaded, embeddings,
// layers, head; normed (host, or null): the last row after the final norm
static int chunk(ihip_mctx* s, const int32_t* ids, const float* embeds, int64_t n,
                 bool want_logits, bool all, uint64_t logits_dev, float* normed, bool first = false)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  ihip_ctx* c = m->c;
  int rc0 = part_start(s, ids ? ids[0] : -1, first);
  if (rc0) return rc0;
  std::vector<float> cs((size_t)n * d.head_dim), cs2((size_t)n * std::max<int64_t>(m->hd2, 1));
  // declared after the host vectors, so destroyed before them: on every early
  // return the queued copies from cs, cs2, ids and embeds have ended first
  struct StreamWait {
    hipStream_t st;
    ~StreamWait() { (void)hipStreamSynchronize(st); }
  } wait_copies{c->stream};
  rotary(d, s->length, n, cs.data());
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs, cs.data(), cs.size() * 4, c->stream));
  if (m->hd2) {
    rotary2(d, m->hd2, s->length, n, cs2.data());
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs2, cs2.data(), cs2.size() * 4, c->stream));
  }
  int rc = s->length == 0 && m->recurrent ? reset_states(s) : 0;
  if (rc) return rc;
  if (ids) {
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->tok, (void*)ids, n * 4, c->stream));
    rc = ihip_enqueue_embed(c, m->embed, m->embed_dt, d.vocab, d.hidden, s->tok, n, s->x);
    if (!rc) rc = embed_scale(s, n);
  } else {
    // ForwardEmbeds: the caller's rows in place of the token embeddings
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->x, (void*)embeds, (size_t)n * d.hidden * 4,
                                  c->stream));
  }
  if (!rc) rc = layers(s, n, s->length, false);
  if (!rc && normed) {
    // one row leaves the residual in x (the head stages the final norm):
    // the norm of that row; a chunk leaves h = the final norm of every row
    uint64_t src = s->h + (uint64_t)(n - 1) * d.hidden * 4;
    if (n == 1 && one_row_fused(m)) {
      rc = ihip_enqueue_rmsnorm(c, s->x, m->final_norm, s->h, 1, d.hidden, d.rms_eps);
      src = s->h;
    }
    if (!rc)
      IHIP_CHECK(hipMemcpyDtoHAsync(normed, (hipDeviceptr_t)src, (size_t)d.hidden * 4, c->stream));
  }
  if (!rc && want_logits) rc = head(s, n, all, logits_dev);
  if (!rc && want_logits) rc = softcap(s, all ? n : 1, logits_dev);
  // the host vectors must outlive the copies
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  if (!rc) {
    for (int64_t i = 0; i < n; i++) s->ids[s->length + i] = ids ? ids[i] : -1;
    s->length += n;
    s->state_ok = true;
  }
  return rc;
}

// the next id from the logits: the argmax, or a draw of the sampler
static int next_token(ihip_mctx* s)
{
  ihip_model* m = s->m;
  const int64_t n = s->draw_ids > 0 ? std::min<int64_t>(s->draw_ids, m->d.vocab) : m->d.vocab;
  return m->sampler ? ihip_enqueue_sample(m->c, m->sampler, s->logits, n, s->next)
                    : ihip_enqueue_argmax(m->c, s->logits, n, s->next);
}

// the decode step as a graph: embed(tok) -> layers(pos) -> head -> next id
static int decode_body(ihip_mctx* s)
{
  ihip_model* m = s->m;
  ihip_ctx* c = m->c;
  int rc = ihip_enqueue_embed(c, m->embed, m->embed_dt, m->d.vocab, m->d.hidden, s->tok, 1, s->x);
  if (!rc) rc = embed_scale(s, 1);
  if (!rc) rc = layers(s, 1, 0, true);
  if (!rc) rc = head(s, 1, false, s->logits);
  if (!rc) rc = softcap(s, 1, s->logits);
  if (!rc) rc = next_token(s);
  if (!rc && c->capturing && s->cs_tab) {
    // the next step's token, position and rotary rows (a pipelined decode
    // enqueues the steps without reading the ids back in between)
    struct {
      const int* next;
      int* tok;
      int* pos;
      float* cs;
      const float* tab;
      float* cs2;
      const float* tab2;
      int32_t rs, rs2, rows, pad;
    } aa = {(const int*)s->next, (int*)s->tok, (int*)s->pos, (float*)s->cs, (const float*)s->cs_tab,
            m->hd2 ? (float*)s->cs2 : nullptr, m->hd2 ? (const float*)s->cs2_tab : nullptr,
            (int32_t)m->d.head_dim, (int32_t)std::max<int64_t>(m->hd2, 0), (int32_t)s->cs_cap, 0};
    rc = launch(c, "decode_advance", dim3(1), dim3(256), &aa);
  }
  return rc;
}

// the rotary table rows of positions [0, upto) (grown to the context's
// capacity + 1 rows; rows already there are kept)
static int cs_table(ihip_mctx* s, int64_t upto)
{
  ihip_model* m = s->m;
  ihip_ctx* c = m->c;
  const int64_t rs = m->d.head_dim, rs2 = m->hd2;
  const int64_t cap = s->capacity + 1;
  if (s->cs_cap < cap) {
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    free_owned(s, s->cs_tab);
    free_owned(s, s->cs2_tab);
    s->cs_rows = s->cs_cap = 0;
    int rc = dalloc_ctx(s, (uint64_t)cap * rs * 4, s->cs_tab);
    if (!rc && rs2 > 0) rc = dalloc_ctx(s, (uint64_t)cap * rs2 * 4, s->cs2_tab);
    if (rc) return rc;
    s->cs_cap = cap;
    s->graph_ready = false;  // the graph holds the table's address
  }
  upto = std::min(upto, s->cs_cap);
  if (upto <= s->cs_rows) return 0;
  const int64_t n = upto - s->cs_rows;
  std::vector<float> t((size_t)(n * rs), 0.f), t2((size_t)std::max<int64_t>(n * rs2, 1), 0.f);
  for (int64_t r = 0; r < n; r++) {
    rotary(m->d, s->cs_rows + r, 1, t.data() + r * rs);
    if (rs2 > 0) rotary2(m->d, rs2, s->cs_rows + r, 1, t2.data() + r * rs2);
  }
  IHIP_CHECK(hipMemcpyHtoD((hipDeviceptr_t)(s->cs_tab + (uint64_t)s->cs_rows * rs * 4), t.data(), t.size() * 4));
  if (rs2 > 0)
    IHIP_CHECK(hipMemcpyHtoD((hipDeviceptr_t)(s->cs2_tab + (uint64_t)s->cs_rows * rs2 * 4), t2.data(),
                             t2.size() * 4));
  s->cs_rows = upto;
  return 0;
}

// the context's decode graph, captured for its capacity (the attention's
// ranges) and the model's sampler; updated in place when the topology allows
static int decode_graph(ihip_mctx* s)
{
  ihip_model* m = s->m;
  ihip_ctx* c = m->c;
  if (c->capturing) return fail(IHIP_E_CAPTURE, "decode graph: the context is capturing");
  IHIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  c->capturing = true;
  int rc = decode_body(s);
  c->capturing = false;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  bool updated = false;
  if (s->exec) {
    hipGraphExecUpdateResult res;
    hipGraphNode_t err_node = nullptr;
    updated = hipGraphExecUpdate(s->exec, g, &err_node, &res) == hipSuccess &&
              res == hipGraphExecUpdateSuccess;
    if (!updated) {
      (void)hipGetLastError();
      (void)hipGraphExecDestroy(s->exec);
      s->exec = nullptr;
    }
  }
  if (s->graph) (void)hipGraphDestroy(s->graph);
  s->graph = g;
  if (!updated) IHIP_CHECK(hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0));
  s->graph_ready = true;
  s->graph_capacity = s->capacity;
  s->graph_sampler = m->sampler_epoch;
  s->graph_draw = s->draw_ids;
  return 0;
}

static int dalloc_ctx(ihip_mctx* s, uint64_t bytes, uint64_t& p)
{
  void* q = nullptr;
  IHIP_CHECK(hipMalloc(&q, bytes ? (bytes + 255) & ~(uint64_t)255 : 256));
  s->owned.push_back((uint64_t)q);
  p = (uint64_t)q;
  return 0;
}

static void free_owned(ihip_mctx* s, uint64_t& p)
{
  if (!p) return;
  for (size_t i = 0; i < s->owned.size(); i++)
    if (s->owned[i] == p) {
      s->owned.erase(s->owned.begin() + i);
      break;
    }
  (void)hipFree((void*)p);
  p = 0;
}

// the most bytes of attention partials a chunk may use: the rows of a chunk
// are cut down so a long context stays within it
static const uint64_t ATTN_PART_MAX = 1ull << 30;

static uint64_t part_bytes(const ihip_model* m, int64_t rows, int64_t keys)
{
  // one row (the decode step): the ranges rounded up to a multiple of 8 at
  // most, as enqueue_attention_one lays them over the XCDs
  const int64_t splits = attention_splits(keys);
  return (uint64_t)m->d.heads * rows * (rows == 1 ? (splits + 7) / 8 * 8 : splits) * (m->max_hd + 2) * 8;
}

// rows of the next chunk after `past` cached tokens, at most `want`
static int64_t chunk_rows(const ihip_mctx* s, int64_t past, int64_t want, const int32_t* ids = nullptr)
{
  int64_t n = std::min(want, s->m->chunk_rows);
  while (n > 1 && part_bytes(s->m, n, past + n) > ATTN_PART_MAX) n = (n + 1) / 2;
  // a recurrent context with restore points: a part ends before every
  // CheckpointId token (ForwardRows, decoder.pas:3191-3243)
  if (ids && s->m->recurrent && s->ckpt_id >= 0 && s->ckpt_max > 0)
    for (int64_t i = 1; i < n; i++)
      if (ids[i] == s->ckpt_id) return i;
  return n;
}

// Prepare (model.qwen3.cuda.pas:856-940): the KV cache grown to hold
// `tokens` (doubled, at least a quarter beyond them and 64, at most the
// model's positions; the cached rows copied over), and the attention
// partials for chunks of up to CHUNK rows over it
static int prepare(ihip_mctx* s, int64_t tokens)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  ihip_ctx* c = m->c;
  const int64_t maxpos = d.max_positions > 0 ? d.max_positions : ((int64_t)1 << 30);
  if (tokens > maxpos)
    return fail(IHIP_E_ARG, "forward: " + std::to_string(tokens) + " tokens exceed the " +
                                std::to_string(maxpos) + " positions");
  if (tokens > s->capacity) {
    int64_t cap = s->capacity * 2;
    if (cap < tokens + tokens / 4) cap = tokens + tokens / 4;
    if (cap < 64) cap = 64;
    if (cap > maxpos) cap = maxpos;
    const uint64_t es = m->kv_f16 ? 2 : 4;
    std::vector<uint64_t> nk(d.layers, 0), nv(d.layers, 0);
    int rc = 0;
    for (int l = 0; l < d.layers && !rc; l++) {
      if (m->L[l].mixer == IHIP_MIXER_DELTANET) continue;  // a state, no rows
      const uint64_t kvw = (uint64_t)(m->L[l].kvh * m->L[l].hd);
      void* a = nullptr;
      void* b = nullptr;
      hipError_t e = hipMalloc(&a, (uint64_t)cap * kvw * es);
      if (e == hipSuccess) e = hipMalloc(&b, (uint64_t)cap * kvw * es);
      nk[l] = (uint64_t)a;
      nv[l] = (uint64_t)b;
      if (e != hipSuccess) {
        rc = hip_fail(e, "KV cache");
        break;
      }
      if (s->length > 0) {
        e = hipMemcpyDtoDAsync((hipDeviceptr_t)nk[l], (hipDeviceptr_t)s->kc[l], s->length * kvw * es,
                               c->stream);
        if (e == hipSuccess)
          e = hipMemcpyDtoDAsync((hipDeviceptr_t)nv[l], (hipDeviceptr_t)s->vc[l],
                                 s->length * kvw * es, c->stream);
        if (e != hipSuccess) rc = hip_fail(e, "KV cache copy");
      }
    }
    (void)hipStreamSynchronize(c->stream);
    if (rc) {
      for (int l = 0; l < d.layers; l++) {
        if (nk[l]) (void)hipFree((void*)nk[l]);
        if (nv[l]) (void)hipFree((void*)nv[l]);
      }
      return rc;
    }
    for (int l = 0; l < (int)s->kc.size(); l++) {
      if (s->kc[l]) (void)hipFree((void*)s->kc[l]);
      if (s->vc[l]) (void)hipFree((void*)s->vc[l]);
    }
    s->kc = nk;
    s->vc = nv;
    s->ids.resize(cap, -1);
    s->capacity = cap;
  }
  // partials for a chunk of up to CHUNK rows over the cache (or fewer rows:
  // chunk_rows), and for the decode step's ranges over the whole capacity
  const uint64_t want = std::max(part_bytes(m, chunk_rows(s, 0, CHUNK), s->capacity),
                                 part_bytes(m, 1, s->capacity));
  if (s->attn_part_bytes < want) {
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    free_owned(s, s->attn_part);
    s->attn_part_bytes = 0;
    int rc = dalloc_ctx(s, want, s->attn_part);
    if (rc) return rc;
    s->attn_part_bytes = want;
    s->graph_ready = false;
  }
  return 0;
}

// steps decode steps from token `first` (not yet in the cache): each one
// graph launch that writes the next id; out_ids[i] the id after step i
static int decode_steps(ihip_mctx* s, int32_t first, int64_t steps, int32_t* out_ids)
{
  ihip_model* m = s->m;
  ihip_ctx* c = m->c;
  int rc = prepare(s, s->length + steps);
  if (rc) return rc;
  // a graph holds this context's cache and ranges: captured again when the
  // cache grew or the sampler changed since
  const bool graphs = m->use_graphs && !m->check_route && m->tape_rows == 0;
  // the graph's last launch advances token, position and rotary rows: the
  // steps of a model without a recurrent state (whose restore points need
  // each id on the host) go out back to back, the ids read once at the end
  static const bool pipeline_on = [] {
    const char* v = getenv("IHIP_DECODE_PIPELINE");
    return !v || atoi(v) != 0;
  }();
  const bool pipelined = pipeline_on && graphs && !m->recurrent && steps > 1;
  if (graphs && (rc = cs_table(s, s->length + steps + 1))) return rc;
  if (graphs && (!s->graph_ready || s->graph_capacity != s->capacity ||
                        s->graph_sampler != m->sampler_epoch || s->graph_draw != s->draw_ids) &&
      (rc = decode_graph(s)))
    return rc;
  std::vector<float> cs(m->d.head_dim), cs2(std::max<int64_t>(m->hd2, 1));
  int32_t tok = first, pos = 0;
  // destroyed before cs, cs2, tok and pos: on an early return the copies
  // queued from them have ended first
  struct StreamWait {
    hipStream_t st;
    ~StreamWait() { (void)hipStreamSynchronize(st); }
  } wait_copies{c->stream};
  if (pipelined) {
    if (s->ids_pinned_n < steps) {
      IHIP_CHECK(hipStreamSynchronize(c->stream));
      if (s->ids_pinned) (void)hipHostFree(s->ids_pinned);
      s->ids_pinned = nullptr;
      s->ids_pinned_n = 0;
      IHIP_CHECK(hipHostMalloc((void**)&s->ids_pinned, (size_t)steps * 4, hipHostMallocDefault));
      s->ids_pinned_n = steps;
    }
    pos = (int32_t)s->length;
    if (m->hd2) {
      rotary2(m->d, m->hd2, pos, 1, cs2.data());
      IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs2, cs2.data(), cs2.size() * 4, c->stream));
    }
    rotary(m->d, pos, 1, cs.data());
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->tok, &tok, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->pos, &pos, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs, cs.data(), cs.size() * 4, c->stream));
    for (int64_t i = 0; i < steps; i++) {
      IHIP_CHECK(hipGraphLaunch(s->exec, c->stream));
      IHIP_CHECK(hipMemcpyDtoHAsync(s->ids_pinned + i, (hipDeviceptr_t)s->next, 4, c->stream));
    }
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    for (int64_t i = 0; i < steps; i++) {
      out_ids[i] = s->ids_pinned[i];
      s->ids[s->length] = tok;
      s->length++;
      tok = out_ids[i];
    }
    s->state_ok = true;
    return 0;
  }
  for (int64_t i = 0; i < steps; i++) {
    pos = (int32_t)s->length;
    if (pos == 0 && m->recurrent && (rc = reset_states(s))) return rc;
    // each step is a forward of one token: its own part
    if ((rc = part_start(s, tok, true))) return rc;
    if (m->hd2) {
      rotary2(m->d, m->hd2, pos, 1, cs2.data());
      IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs2, cs2.data(), cs2.size() * 4, c->stream));
    }
    rotary(m->d, pos, 1, cs.data());
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->tok, &tok, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->pos, &pos, 4, c->stream));
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)s->cs, cs.data(), cs.size() * 4, c->stream));
    if (graphs) {
      IHIP_CHECK(hipGraphLaunch(s->exec, c->stream));
    } else if ((rc = decode_body(s))) {
      return rc;
    }
    IHIP_CHECK(hipMemcpyDtoHAsync(&out_ids[i], (hipDeviceptr_t)s->next, 4, c->stream));
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    s->ids[s->length] = tok;
    s->length++;
    s->state_ok = true;
    tok = out_ids[i];
  }
  return 0;
}

static void context_free(ihip_mctx* s)
{
  if (!s) return;
  ihip_ctx* c = s->m->c;
  (void)hipStreamSynchronize(c->stream);
  if (s->ids_pinned) (void)hipHostFree(s->ids_pinned);
  if (s->exec) (void)hipGraphExecDestroy(s->exec);
  if (s->graph) (void)hipGraphDestroy(s->graph);
  for (auto p : s->owned) (void)hipFree((void*)p);
  if (s->logits_all) (void)hipFree((void*)s->logits_all);
  for (size_t l = 0; l < s->kc.size(); l++) {
    if (s->kc[l]) (void)hipFree((void*)s->kc[l]);
    if (s->vc[l]) (void)hipFree((void*)s->vc[l]);
  }
  delete s;
}

// a new context: the activations of one chunk, the attention counters, and a
// KV cache of `capacity` tokens (0: none until the first tokens come)
static int context_new(ihip_model* m, int64_t capacity, ihip_mctx** out)
{
  *out = nullptr;
  ihip_mctx* s = new ihip_mctx();
  s->m = m;
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden, hd = m->max_hd, qw = m->max_qw, kvw = m->max_kvw;
  const int64_t N = CHUNK;
  int64_t F = std::max<int64_t>(d.ffn, 1);
  int64_t EK = m->any_moe ? (int64_t)d.experts_used * d.expert_ffn : 0;
  int64_t wide = std::max<int64_t>({F, EK, qw, H, (int64_t)d.experts});
  const int64_t K1 = std::max(d.experts_used, 1), E1 = std::max(d.experts, 1);
  const int64_t lvd = (int64_t)d.lin_value_heads * d.lin_value_dim,
                lcd = 2 * (int64_t)d.lin_key_heads * d.lin_key_dim + lvd;
  const uint64_t qin = std::max<int64_t>({H, qw, F, (int64_t)d.expert_ffn, lvd});
  const uint64_t qrow = qin + 4 * (qin / 32);
  int rc = 0;
  auto bad = [&](int r) {
    context_free(s);
    return r;
  };
  s->kc.assign(d.layers, 0);
  s->vc.assign(d.layers, 0);
  if ((rc = dalloc_ctx(s, N * H * 4, s->x)) || (rc = dalloc_ctx(s, N * H * 4, s->h)) ||
      (rc = dalloc_ctx(s, N * H * 4, s->tmp)) || (rc = dalloc_ctx(s, N * qw * 4, s->q)) ||
      (rc = dalloc_ctx(s, N * kvw * 4, s->k)) || (rc = dalloc_ctx(s, N * kvw * 4, s->v)) ||
      (rc = dalloc_ctx(s, N * qw * 4, s->attn)) || (rc = dalloc_ctx(s, N * wide * 4, s->gate)) ||
      (rc = dalloc_ctx(s, N * wide * 4, s->up)) || (rc = dalloc_ctx(s, N * E1 * 4, s->route)) ||
      (rc = dalloc_ctx(s, N * K1 * 4, s->ids_dev)) || (rc = dalloc_ctx(s, N * K1 * 4, s->rw)) ||
      (rc = dalloc_ctx(s, N * K1 * H * 4, s->eout)) || (rc = dalloc_ctx(s, N * hd * 4, s->cs)) ||
      (rc = dalloc_ctx(s, N * 4, s->tok)) || (rc = dalloc_ctx(s, (uint64_t)d.vocab * 4, s->logits)) ||
      (rc = dalloc_ctx(s, 256, s->next)) || (rc = dalloc_ctx(s, 256, s->pos)) ||
      (rc = dalloc_ctx(s, N * K1 * 4, s->perm)) ||
      (rc = dalloc_ctx(s, (N * K1 / 8 + 1 + E1) * 16, s->items)) ||
      (rc = dalloc_ctx(s, N * qrow, s->xq0)) || (rc = dalloc_ctx(s, N * qrow, s->xqk)) ||
      (rc = dalloc_ctx(s, N * K1 * qrow, s->xqf)) || (rc = dalloc_ctx(s, 256 * 128, s->done)))
    return bad(rc);
  s->conv.assign(d.layers, 0);
  s->state.assign(d.layers, 0);
  if (m->recurrent) {
    const int64_t lvh = std::max(d.lin_value_heads, 1);
    if ((rc = dalloc_ctx(s, N * lcd * 4, s->qkv)) || (rc = dalloc_ctx(s, N * lvd * 4, s->z)) ||
        (rc = dalloc_ctx(s, N * lvh * 4, s->beta)) || (rc = dalloc_ctx(s, N * lvh * 4, s->decay)) ||
        (rc = dalloc_ctx(s, N * lvd * 4, s->core)))
      return bad(rc);
    for (int l = 0; l < d.layers; l++)
      if (m->L[l].mixer == IHIP_MIXER_DELTANET &&
          ((rc = dalloc_ctx(s, lcd * std::max(d.lin_conv - 1, 1) * 4, s->conv[l])) ||
           (rc = dalloc_ctx(s, lvd * d.lin_key_dim * 4, s->state[l]))))
        return bad(rc);
  }
  if (m->gated && ((rc = dalloc_ctx(s, N * 2 * qw * 4, s->qg)) || (rc = dalloc_ctx(s, N * qw * 4, s->gq))))
    return bad(rc);
  if (m->hd2 > 0 && (rc = dalloc_ctx(s, N * m->hd2 * 4, s->cs2))) return bad(rc);
  if (m->gemma && (rc = dalloc_ctx(s, N * H * 4, s->moe))) return bad(rc);
  // the attention counters start at zero (a fill kernel would do under
  // capture; this runs once, outside any capture)
  {
    const hipError_t e = hipMemsetAsync((void*)s->done, 0, 256 * 128, m->c->stream);
    if (e != hipSuccess) return bad(hip_fail(e, "model: counters"));
  }
  if (capacity > 0 && (rc = prepare(s, capacity))) return bad(rc);
  m->contexts.push_back(s);
  *out = s;
  return 0;
}

// TDecoderModel.Forward / ForwardEmbeds on a context (ForwardRows,
// model.qwen3.cuda.pas:1656-1720): chunks of the rows, logits of the last
// row (or of every row), the last row's final norm into normed
static int context_forward(ihip_mctx* s, const int32_t* ids, const float* embeds, int64_t count,
                           float* logits, int all_logits, float* normed, int head_index)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  if (count < 1 || (!ids && !embeds)) return fail(IHIP_E_ARG, "forward: no tokens");
  if (head_index != 0) return fail(IHIP_E_ARG, "forward: no head " + std::to_string(head_index) + " (1 head)");
  if (ids)
    for (int64_t i = 0; i < count; i++)
      if (ids[i] < 0 || ids[i] >= d.vocab)
        return fail(IHIP_E_ARG, "forward: token id " + std::to_string(ids[i]) + " outside the vocabulary");
  std::lock_guard<std::mutex> g(m->c->lock);
  int rc = prepare(s, s->length + count);
  if (rc) return rc;
  for (int64_t done = 0; done < count;) {
    const int64_t n = chunk_rows(s, s->length, count - done, ids ? ids + done : nullptr);
    const bool last = done + n == count;
    const bool want = logits && (all_logits || last);
    uint64_t ldev = s->logits;
    if (want && all_logits) {
      if (s->logits_all_rows < n) {
        if (s->logits_all) (void)hipFree((void*)s->logits_all);
        s->logits_all = 0;
        s->logits_all_rows = 0;
        void* p = nullptr;
        IHIP_CHECK(hipMalloc(&p, (uint64_t)CHUNK * d.vocab * 4));
        s->logits_all = (uint64_t)p;
        s->logits_all_rows = CHUNK;
      }
      ldev = s->logits_all;
    }
    rc = chunk(s, ids ? ids + done : nullptr, embeds ? embeds + done * d.hidden : nullptr, n, want,
               all_logits != 0, ldev, last ? normed : nullptr, done == 0);
    if (rc) return rc;
    if (want) {
      float* dst = all_logits ? logits + done * d.vocab : logits;
      const uint64_t rows = all_logits ? n : 1;
      IHIP_CHECK(hipMemcpyDtoHAsync(dst, (hipDeviceptr_t)ldev, rows * d.vocab * 4, m->c->stream));
      IHIP_CHECK(hipStreamSynchronize(m->c->stream));
    }
    done += n;
  }
  return 0;
}

// TDecoderModel.Greedy (decoder.pas:3390-3426) on a context
static int context_greedy(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                          int32_t* out_ids)
{
  ihip_model* m = s->m;
  ihip_ctx* c = m->c;
  for (int64_t i = 0; i < n; i++)
    if (prompt[i] < 0 || prompt[i] >= m->d.vocab) return fail(IHIP_E_ARG, "greedy: token id outside the vocabulary");
  auto t0 = std::chrono::steady_clock::now();
  int rc = 0;
  {
    // the prompt: every chunk, logits of the last row only, argmax on device
    std::lock_guard<std::mutex> g(c->lock);
    if ((rc = prepare(s, s->length + n + max_new))) return rc;
    for (int64_t done = 0; done < n && !rc;) {
      const int64_t k = chunk_rows(s, s->length, n - done, prompt + done);
      rc = chunk(s, prompt + done, nullptr, k, done + k == n, false, s->logits, nullptr, done == 0);
      done += k;
    }
    if (!rc) rc = next_token(s);
    if (!rc) {
      IHIP_CHECK(hipMemcpyDtoHAsync(&out_ids[0], (hipDeviceptr_t)s->next, 4, c->stream));
      IHIP_CHECK(hipStreamSynchronize(c->stream));
    }
  }
  if (rc) return rc;
  auto t1 = std::chrono::steady_clock::now();
  std::lock_guard<std::mutex> g(c->lock);
  // the new ids, then the last one into the cache too (TDecoderModel.Greedy:
  // a Forward without logits after the last step), through the same graph
  if (max_new > 1 && (rc = decode_steps(s, out_ids[0], max_new - 1, out_ids + 1))) return rc;
  int32_t spare;
  if ((rc = decode_steps(s, out_ids[max_new - 1], 1, &spare))) return rc;
  auto t2 = std::chrono::steady_clock::now();
  s->prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  s->decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  return 0;
}

static int context_decode(ihip_mctx* s, int32_t first, int64_t steps, int32_t* out_ids)
{
  if (first < 0 || first >= s->m->d.vocab) return fail(IHIP_E_ARG, "decode: token id outside the vocabulary");
  std::lock_guard<std::mutex> g(s->m->c->lock);
  auto t0 = std::chrono::steady_clock::now();
  int rc = decode_steps(s, first, steps, out_ids);
  s->decode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  return rc;
}

// ---------------------------------------------------------------------
// TNativeLlmClient's device side (src/mormot.ai.llm.native.pas): NativeDecode
// (:2135-2185), one request on a context, and TNativePromptCache
// (:2192-2350), the contexts kept between requests for their prompts. The
// tokenizer, chat template and output parser stay the caller's: the parser's
// stop is a set of token ids here.

// the cached tokens of s that start prompt, at most count of them (a position
// fed an embedding row matches no id): TDecoderContext.Usable
static int64_t usable(const ihip_mctx* s, const int32_t* prompt, int64_t count)
{
  int64_t n = 0;
  const int64_t lim = std::min<int64_t>(std::max<int64_t>(count, 0), s->length);
  while (n < lim && s->ids[n] >= 0 && s->ids[n] == prompt[n]) n++;
  // a recurrent state holds the whole sequence: all of it, else the last
  // restore point before the end of the common start whose token is the
  // prompt's CheckpointId token there too (TDecoderContext.Usable,
  // decoder.pas:1213-1230)
  if (!s->m->recurrent || n == 0 || (n == s->length && s->state_ok)) return n;
  const int64_t prefix = n;
  n = 0;
  for (auto& c : s->ckpts)
    if (c.first < prefix && s->ids[c.first] == s->ckpt_id && c.first > n && restorable(s, c.first)) n = c.first;
  return n;
}

// the draws of a request from a fresh TInferSampler: the model's sampler kept
// when its settings are the request's (its stream restarted at the seed, the
// decode graphs kept), else replaced (the graphs captured again)
int model_sampling_locked(ihip_model* m, const ihip_sampling* s);

// called with the device lock held, so a request's sampler cannot be swapped
// or reseeded by another context's request before its decode has drawn
static int request_sampler(ihip_model* m, const ihip_sampling* smp)
{
  const bool greedy = !smp || !(smp->temperature > 0);
  if (greedy) return m->sampler || smp ? model_sampling_locked(m, smp) : 0;
  ihip_sampler* k = m->sampler;
  if (k && k->temperature == smp->temperature && k->top_k == smp->top_k && k->top_p == smp->top_p &&
      k->min_p == smp->min_p) {
    const uint64_t seed = (uint64_t)smp->seed;
    IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)k->state, (void*)&seed, 8, m->c->stream));
    IHIP_CHECK(hipStreamSynchronize(m->c->stream));
    return 0;
  }
  return model_sampling_locked(m, smp);
}

static int native_decode(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                         const ihip_sampling* smp, int64_t draw_ids, const int32_t* stop,
                         int64_t nstop, int64_t max_context, int32_t* out_ids, int64_t* out_count,
                         int64_t* reused, int* stopped)
{
  ihip_model* m = s->m;
  const ihip_model_desc& d = m->d;
  int64_t limit = d.max_positions > 0 ? d.max_positions : INT64_MAX;
  if (max_context > 0 && max_context < limit) limit = max_context;
  if (n < 1) return fail(IHIP_E_ARG, "NativeDecode: empty prompt");
  if (n > limit)
    return fail(IHIP_E_ARG, "NativeDecode: a prompt of " + std::to_string(n) +
                                " tokens exceeds the context of " + std::to_string(limit));
  if (max_new <= 0) return fail(IHIP_E_ARG, "NativeDecode: " + std::to_string(max_new) + " new tokens");
  for (int64_t i = 0; i < n; i++)
    if (prompt[i] < 0 || prompt[i] >= d.vocab) return fail(IHIP_E_ARG, "NativeDecode: token id outside the vocabulary");
  // token k is fed at position n + k - 1 only when another one follows
  if (max_new > limit - n + 1) max_new = limit - n + 1;
  // one lock over the sampler's set-up and the whole decode: a request of
  // another context of this model waits, so it cannot change this one's draws
  std::lock_guard<std::mutex> g(m->c->lock);
  int rc = request_sampler(m, smp);
  if (rc) return rc;
  s->draw_ids = draw_ids > 0 && draw_ids < d.vocab ? draw_ids : 0;
  // the cached start of the prompt stays, the rest is computed
  const int64_t kept = usable(s, prompt, n - 1);
  if ((rc = truncate_to(s, kept))) return rc;
  if ((rc = prepare(s, n + max_new))) return rc;
  for (int64_t done = kept; done < n && !rc;) {
    const int64_t k = chunk_rows(s, s->length, n - done, prompt + done);
    rc = chunk(s, prompt + done, nullptr, k, done + k == n, false, s->logits, nullptr, done == kept);
    done += k;
  }
  if (!rc) rc = next_token(s);
  if (rc) return rc;
  int32_t id = 0;
  IHIP_CHECK(hipMemcpyDtoHAsync(&id, (hipDeviceptr_t)s->next, 4, m->c->stream));
  IHIP_CHECK(hipStreamSynchronize(m->c->stream));
  int64_t count = 0;
  bool stop_hit = false;
  for (;;) {
    out_ids[count++] = id;
    for (int64_t i = 0; i < nstop && !stop_hit; i++) stop_hit = stop[i] == id;
    if (stop_hit || count == max_new) break;
    int32_t next = 0;
    if ((rc = decode_steps(s, id, 1, &next))) return rc;
    id = next;
  }
  *out_count = count;
  if (reused) *reused = kept;
  if (stopped) *stopped = stop_hit ? 1 : 0;
  return 0;
}

}  // namespace ihip

// the contexts kept between requests, least recently used first
struct ihip_prompt_cache {
  ihip_model* m = nullptr;
  int64_t slots = 0;
  std::mutex mu;
  std::vector<ihip_mctx*> idle;
  int64_t requests = 0, hits = 0, reused = 0;
};

namespace ihip {
}  // namespace ihip

namespace ihip {
// ihip_model_sampling with the device lock already held by the caller
int model_sampling_locked(ihip_model* m, const ihip_sampling* s)
{
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
  m->sampler_epoch++;  // every context's decode graph is captured again with it
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
  const ihip_model_desc& d = m->d;
  const int64_t H = d.hidden;
  int rc = 0;
  auto bad = [&](int r) {
    ihip_model_destroy(m);
    return r;
  };
  m->gemma = d.activation != IHIP_ACT_SILU || d.value_norm || d.embed_scale > 0 || d.logit_softcap > 0 ||
             d.attention_scale > 0;
  m->max_hd = d.head_dim;
  m->max_qw = (int64_t)d.heads * d.head_dim;
  m->max_kvw = (int64_t)d.kv_heads * d.head_dim;
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
  bool& any_moe = m->any_moe;
  for (int l = 0; l < d.layers; l++) {
    const ihip_layer_desc& s = m->layer_desc[l];
    DevLayer& L = m->L[l];
    // this layer's heads (Gemma 4: its own per layer)
    const int64_t hd = s.head_dim > 0 ? s.head_dim : d.head_dim;
    const int64_t kvh = s.kv_heads > 0 ? s.kv_heads : d.kv_heads;
    const int64_t qw = (int64_t)d.heads * hd, kvw = kvh * hd;
    L.hd = hd;
    L.kvh = kvh;
    L.k_is_v = s.k_is_v != 0;
    L.rope_set = s.rope_set != 0;
    L.no_rope = s.no_rope != 0;
    if (kvh < 1 || d.heads % kvh || (hd & 1) || hd < 2 || hd > 512)
      return bad(fail(IHIP_E_ARG, "model: layer " + std::to_string(l) + " has heads of " + std::to_string(hd) +
                                      " with " + std::to_string(kvh) + " KV heads (even, up to 512)"));
    if (s.head_dim > 0 || s.kv_heads > 0 || s.k_is_v || s.rope_set || s.attn_out_norm.data || s.ffn_out_norm.data ||
        s.scalar.data || s.moe == IHIP_FFN_DENSE_MOE || s.exp_gate_up)
      m->gemma = true;
    if (s.mixer != IHIP_MIXER_DELTANET) {
      m->max_hd = std::max(m->max_hd, hd);
      m->max_qw = std::max(m->max_qw, qw);
      m->max_kvw = std::max(m->max_kvw, kvw);
      if (L.rope_set) {
        if (m->hd2 && m->hd2 != hd)
          return bad(fail(IHIP_E_ARG, "model: layers of the second rotary set with heads of two sizes"));
        m->hd2 = hd;
      }
    }
    if ((rc = upf(m, s.attn_out_norm, H, L.attn_out_norm)) || (rc = upf(m, s.ffn_out_norm, H, L.ffn_out_norm)) ||
        (rc = upf(m, s.scalar, 1, L.scalar)))
      return bad(rc);
    L.window = s.window;
    L.moe = s.moe;
    L.mixer = s.mixer;
    L.output_gate = s.output_gate != 0;
    any_moe |= s.moe != 0;
    if (s.mixer != IHIP_MIXER_ATTENTION && s.mixer != IHIP_MIXER_DELTANET)
      return bad(fail(IHIP_E_ARG, "model: layer " + std::to_string(l) + " has an unknown mixer"));
    if (s.mixer == IHIP_MIXER_DELTANET) {
      // Qwen3.5's Gated DeltaNet (model.qwen35.pas:552-590)
      const int64_t vh = d.lin_value_heads, vd = vh * d.lin_value_dim,
                    cd = 2 * (int64_t)d.lin_key_heads * d.lin_key_dim + vd;
      m->recurrent = true;
      if ((rc = upf(m, s.input_norm, H, L.input_norm)) || (rc = upf(m, s.post_norm, H, L.post_norm)) ||
          (rc = upw(m, s.lin_qkv, cd, H, 1, L.lqkv, L.lqkvd)) || (rc = upw(m, s.lin_z, vd, H, 1, L.lz, L.lzd)) ||
          (rc = upw(m, s.lin_b, vh, H, 1, L.lb, L.lbd)) || (rc = upw(m, s.lin_a, vh, H, 1, L.la, L.lad)) ||
          (rc = upw(m, s.lin_out, H, vd, 1, L.lout, L.loutd)) ||
          (rc = upf(m, s.lin_conv, cd * d.lin_conv, L.lconv)) || (rc = upf(m, s.lin_dt_bias, vh, L.ldt)) ||
          (rc = upf(m, s.lin_neg_a, vh, L.lnega)) || (rc = upf(m, s.lin_norm, d.lin_value_dim, L.lnorm)) ||
          (rc = upw(m, s.gate, d.ffn, H, 1, L.gate, L.gd)) || (rc = upw(m, s.up, d.ffn, H, 1, L.up, L.ud)) ||
          (rc = upw(m, s.down, H, d.ffn, 1, L.down, L.dd)))
        return bad(rc);
      if (!L.lqkv || !L.lz || !L.lb || !L.la || !L.lout || !L.lconv || !L.ldt || !L.lnega || !L.lnorm ||
          s.moe)
        return bad(fail(IHIP_E_ARG, "model: DeltaNet layer " + std::to_string(l) + " lacks a tensor"));
      if (s.lin_b.dtype == s.lin_a.dtype) {
        // beta's rows then alpha's as one matrix: the one-row path reads both
        // in the launch of the other projections
        const uint64_t rb = row_bytes(s.lin_b.dtype, H) * vh;
        auto buf = std::make_unique<std::vector<uint8_t>>(2 * rb);
        memcpy(buf->data(), s.lin_b.data, rb);
        memcpy(buf->data() + rb, s.lin_a.data, rb);
        const ihip_tensor t{buf->data(), s.lin_b.dtype, 0};
        m->host_owned.push_back(std::move(buf));
        if ((rc = upw(m, t, 2 * vh, H, 1, L.lba, L.lbad))) return bad(rc);
      }
      continue;
    }
    m->gated |= L.output_gate != 0;
    if ((rc = upf(m, s.input_norm, H, L.input_norm)) || (rc = upf(m, s.post_norm, H, L.post_norm)) ||
        (rc = upw(m, s.q, L.output_gate ? 2 * qw : qw, H, 1, L.q, L.qd)) ||
        (rc = upw(m, s.k, kvw, H, 1, L.k, L.kd)) ||
        (rc = upw(m, s.v, kvw, H, 1, L.v, L.vd)) || (rc = upw(m, s.o, H, qw, 1, L.o, L.od)) ||
        (rc = upf(m, s.q_bias, qw, L.qb)) || (rc = upf(m, s.k_bias, kvw, L.kb)) ||
        (rc = upf(m, s.v_bias, kvw, L.vb)) || (rc = upf(m, s.o_bias, H, L.ob)) ||
        (rc = upf(m, s.q_norm, hd, L.qn)) || (rc = upf(m, s.k_norm, hd, L.kn)) ||
        (rc = upf(m, s.sinks, d.heads, L.sinks)))
      return bad(rc);
    if (s.moe != IHIP_FFN_MOE) {
      if ((rc = upw(m, s.gate, d.ffn, H, 1, L.gate, L.gd)) || (rc = upw(m, s.up, d.ffn, H, 1, L.up, L.ud)) ||
          (rc = upw(m, s.down, H, d.ffn, 1, L.down, L.dd)))
        return bad(rc);
    }
    if (s.moe != IHIP_FFN_DENSE) {
      const int64_t E = d.experts, FI = d.expert_ffn;
      if (s.exp_gate_up) {
        // [E, 2 FI, H], per expert its gate rows then its up rows: uploaded
        // as two matrices of FI rows per expert
        if (!s.exp_gate.data) return bad(fail(IHIP_E_ARG, "experts: no gate_up tensor"));
        const uint64_t rb = row_bytes(s.exp_gate.dtype, H);
        m->uploaded.emplace_back((const uint8_t*)s.exp_gate.data, rb * 2 * FI * E);
        L.egd = L.eud = s.exp_gate.dtype;
        if ((rc = weight_rows(c, s.exp_gate.data, L.egd, FI, H, E, 2 * FI, &L.eg)) ||
            (rc = weight_rows(c, (const uint8_t*)s.exp_gate.data + rb * FI, L.eud, FI, H, E, 2 * FI, &L.eu)))
          return bad(rc);
      } else if ((rc = upw(m, s.exp_gate, FI, H, E, L.eg, L.egd)) || (rc = upw(m, s.exp_up, FI, H, E, L.eu, L.eud))) {
        return bad(rc);
      }
      if ((rc = upw(m, s.router, E, H, 1, L.router, L.rd)) || (rc = upf(m, s.router_bias, E, L.router_b)) ||
          (rc = upw(m, s.exp_down, H, FI, E, L.ed, L.edd)) ||
          (rc = upf(m, s.dense_out_norm, H, L.dense_out_norm)) || (rc = upf(m, s.moe_in_norm, H, L.moe_in_norm)) ||
          (rc = upf(m, s.moe_out_norm, H, L.moe_out_norm)) || (rc = upf(m, s.router_norm, H, L.router_norm)) ||
          (rc = upf(m, s.expert_scale, E, L.expert_scale)) ||
          (rc = upf(m, s.exp_gate_bias, E * FI, L.egb)) ||
          (rc = upf(m, s.exp_up_bias, E * FI, L.eub)) ||
          (rc = upf(m, s.exp_down_bias, E * H, L.edb)))
        return bad(rc);
      if (L.egd != L.eud) return bad(fail(IHIP_E_ARG, "experts: gate and up of one type"));
      L.eg_stride = (int64_t)row_bytes(L.egd, H) * FI;
      L.ed_stride = (int64_t)row_bytes(L.edd, FI) * H;
    }
  }
  const int64_t hd = d.head_dim;
  if ((hd & 1) || hd > 512) return bad(fail(IHIP_E_ARG, "model: an odd head size or one beyond 512"));
  const int64_t rot = rope_dims(d);
  if (rot < 2 || rot > hd || (rot & 1)) return bad(fail(IHIP_E_ARG, "model: an odd or oversized rotary share"));
  if (m->hd2 && (d.rope2_pairs < 1 || d.rope2_pairs > m->hd2 / 2 || !(d.rope2_theta > 1)))
    return bad(fail(IHIP_E_ARG, "model: the second rotary set's pairs or theta"));
  // the DeltaNet kernels keep a state column in a wave's registers (keys of
  // up to 256) and the convolution inputs in a thread's (up to 8)
  if (m->recurrent &&
      (d.lin_key_heads < 1 || d.lin_value_heads < d.lin_key_heads || d.lin_value_heads % d.lin_key_heads ||
       d.lin_key_dim < 1 || d.lin_key_dim > 256 || d.lin_value_dim < 1 || d.lin_value_dim > 1024 ||
       d.lin_conv < 1 || d.lin_conv > 8))
    return bad(fail(IHIP_E_UNSUPPORTED, "model: DeltaNet shapes beyond the device kernels (keys <= 256, "
                                        "convolution <= 8)"));
  // moe_plan counts the slots per expert in LDS (4096 experts); a chunk's
  // work items stay within one grid dimension
  if (any_moe && (d.experts > 4096 || CHUNK * d.experts_used > 65535))
    return bad(fail(IHIP_E_ARG, "model: more than 4096 experts or 65535 slots per chunk"));
  // a prompt chunk's experts on the MFMA GEMM when every expert matrix can
  // run there: work items of 64 slots
  bool all_gemm = any_moe;
  for (const DevLayer& L : m->L)
    if (L.moe)
      all_gemm = all_gemm && gemm_runs(c, L.egd, mode) && gemm_runs(c, L.eud, mode) &&
                 gemm_runs(c, L.edd, mode);
  m->item_rows = all_gemm ? 64 : 8;
  // the model's own context, its cache sized for max_tokens up front
  if ((rc = context_new(m, max_tokens, &m->def))) return bad(rc);
  m->def->is_default = true;
  *out = m;
  return 0;
}

void ihip_model_destroy(ihip_model* m)
{
  if (!m) return;
  (void)hipStreamSynchronize(m->c->stream);
  for (ihip_mctx* s : m->contexts) context_free(s);
  m->contexts.clear();
  ihip_sampler_destroy(m->sampler);
  for (auto& u : m->uploaded) ihip_forget_weights(m->c, u.first, u.first + u.second);
  delete m;
}

int ihip_model_reset(ihip_model* m)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_reset");
  std::lock_guard<std::mutex> g(m->c->lock);
  return truncate_to(m->def, 0);
}

int ihip_context_set_checkpoints(ihip_mctx* s, int32_t id, int64_t max)
{
  if (!s || max < 0) return fail(IHIP_E_ARG, "ihip_context_set_checkpoints");
  std::lock_guard<std::mutex> g(s->m->c->lock);
  // SetCheckpointId / SetMaxCheckpoints (decoder.pas:1019-1047): another id
  // drops the restore points (the rows cached were split by the old one);
  // a smaller count drops the oldest
  if (id != s->ckpt_id) {
    s->ckpt_id = id;
    s->ckpts.clear();
    s->aligned = s->length == 0;
  }
  s->ckpt_max = max;
  while ((int64_t)s->ckpts.size() > max) s->ckpts.erase(s->ckpts.begin());
  return 0;
}

int ihip_context_checkpoints(ihip_mctx* s, int64_t* lengths, int64_t cap, int64_t* count)
{
  if (!s || !count || (cap > 0 && !lengths)) return fail(IHIP_E_ARG, "ihip_context_checkpoints");
  std::lock_guard<std::mutex> g(s->m->c->lock);
  *count = (int64_t)s->ckpts.size();
  for (int64_t i = 0; i < *count && i < cap; i++) lengths[i] = s->ckpts[i].first;
  return 0;
}

int ihip_model_forward(ihip_model* m, const int32_t* ids, int64_t count, float* logits,
                       int all_logits)
{
  if (!m || !ids || count < 1) return fail(IHIP_E_ARG, "ihip_model_forward: no tokens");
  return context_forward(m->def, ids, nullptr, count, logits, all_logits, nullptr, 0);
}

int ihip_model_greedy(ihip_model* m, const int32_t* prompt, int64_t n, int64_t max_new,
                      int32_t* out_ids)
{
  if (!m || !prompt || n < 1 || max_new < 1 || !out_ids) return fail(IHIP_E_ARG, "ihip_model_greedy");
  return context_greedy(m->def, prompt, n, max_new, out_ids);
}

int ihip_model_decode(ihip_model* m, int32_t first, int64_t steps, int32_t* out_ids)
{
  if (!m || steps < 1 || !out_ids) return fail(IHIP_E_ARG, "ihip_model_decode");
  return context_decode(m->def, first, steps, out_ids);
}

/* ---- contexts (TDecoderDevice.NewDeviceContext and the calls on one) ---- */

int ihip_model_new_context(ihip_model* m, ihip_mctx** out)
{
  if (!m || !out) return fail(IHIP_E_ARG, "ihip_model_new_context");
  std::lock_guard<std::mutex> g(m->c->lock);
  return context_new(m, 0, out);
}

void ihip_context_destroy(ihip_mctx* s)
{
  if (!s || s->is_default) return;  // the model's own context goes with the model
  ihip_model* m = s->m;
  std::lock_guard<std::mutex> g(m->c->lock);
  for (size_t i = 0; i < m->contexts.size(); i++)
    if (m->contexts[i] == s) {
      m->contexts.erase(m->contexts.begin() + i);
      break;
    }
  context_free(s);
}

ihip_mctx* ihip_model_context(ihip_model* m) { return m ? m->def : nullptr; }

int ihip_context_forward(ihip_mctx* s, const int32_t* ids, int64_t count, float* logits,
                         int all_logits)
{
  if (!s || !ids || count < 1) return fail(IHIP_E_ARG, "ihip_context_forward: no ids");
  return context_forward(s, ids, nullptr, count, logits, all_logits, nullptr, 0);
}

int ihip_context_forward_embeds(ihip_mctx* s, const float* embeds, int64_t count, float* logits,
                                int all_logits, float* normed, int head)
{
  if (!s || !embeds || count < 1) return fail(IHIP_E_ARG, "ihip_context_forward_embeds: no rows");
  return context_forward(s, nullptr, embeds, count, logits, all_logits, normed, head);
}

int ihip_context_truncate(ihip_mctx* s, int64_t length)
{
  if (!s || length < 0 || length > s->length)
    return fail(IHIP_E_ARG, "ihip_context_truncate(" + std::to_string(length) + ") of " +
                                std::to_string(s ? s->length : 0) + " tokens");
  // the cache keeps every row: any length but where a DeltaNet state cannot
  // go back (to 0 or a restore point only)
  std::lock_guard<std::mutex> g(s->m->c->lock);
  return truncate_to(s, length);
}

int ihip_context_reuse(ihip_mctx* s, const int32_t* ids, int64_t count, int64_t* kept)
{
  if (!s || (!ids && count > 0) || !kept) return fail(IHIP_E_ARG, "ihip_context_reuse");
  // the common prefix, at most count - 1 tokens (the last one is computed
  // again for its logits); a position fed an embedding row matches no id
  std::lock_guard<std::mutex> g(s->m->c->lock);
  const int64_t n = usable(s, ids, count > 0 ? count - 1 : 0);
  int rc = truncate_to(s, n);
  if (rc) return rc;
  *kept = n;
  return 0;
}

int ihip_context_length(ihip_mctx* s, int64_t* length, int64_t* capacity)
{
  if (!s) return fail(IHIP_E_ARG, "ihip_context_length");
  if (length) *length = s->length;
  if (capacity) *capacity = s->capacity;
  return 0;
}

int ihip_context_greedy(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                        int32_t* out_ids)
{
  if (!s || !prompt || n < 1 || max_new < 1 || !out_ids) return fail(IHIP_E_ARG, "ihip_context_greedy");
  return context_greedy(s, prompt, n, max_new, out_ids);
}

int ihip_context_decode(ihip_mctx* s, int32_t first, int64_t steps, int32_t* out_ids)
{
  if (!s || steps < 1 || !out_ids) return fail(IHIP_E_ARG, "ihip_context_decode");
  return context_decode(s, first, steps, out_ids);
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
  return model_sampling_locked(m, s);
}

int ihip_native_decode(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                       const ihip_sampling* sampling, int64_t draw_ids, const int32_t* stop_ids,
                       int64_t nstop, int64_t max_context, int32_t* out_ids, int64_t* out_count,
                       int64_t* reused, int* stopped)
{
  if (!s || (!prompt && n > 0) || !out_ids || !out_count || nstop < 0 || (nstop > 0 && !stop_ids))
    return fail(IHIP_E_ARG, "ihip_native_decode");
  *out_count = 0;
  return native_decode(s, prompt, n, max_new, sampling, draw_ids, stop_ids, nstop, max_context,
                       out_ids, out_count, reused, stopped);
}

int ihip_prompt_cache_create(ihip_model* m, int64_t slots, ihip_prompt_cache** out)
{
  if (!m || !out || slots < 0) return fail(IHIP_E_ARG, "ihip_prompt_cache_create");
  auto* pc = new ihip_prompt_cache;
  pc->m = m;
  pc->slots = slots;
  *out = pc;
  return 0;
}

static void free_contexts(std::vector<ihip_mctx*>& drop)
{
  for (ihip_mctx* x : drop) ihip_context_destroy(x);
  drop.clear();
}

void ihip_prompt_cache_destroy(ihip_prompt_cache* pc)
{
  if (!pc) return;
  free_contexts(pc->idle);
  delete pc;
}

int ihip_prompt_cache_set_slots(ihip_prompt_cache* pc, int64_t slots)
{
  if (!pc || slots < 0) return fail(IHIP_E_ARG, "ihip_prompt_cache_set_slots");
  std::vector<ihip_mctx*> drop;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    pc->slots = slots;
    const int64_t n = (int64_t)pc->idle.size() - slots;
    if (n > 0) {  // the least recently used go
      drop.assign(pc->idle.begin(), pc->idle.begin() + n);
      pc->idle.erase(pc->idle.begin(), pc->idle.begin() + n);
    }
  }
  free_contexts(drop);
  return 0;
}

int ihip_prompt_cache_clear(ihip_prompt_cache* pc)
{
  if (!pc) return fail(IHIP_E_ARG, "ihip_prompt_cache_clear");
  std::vector<ihip_mctx*> drop;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    drop.swap(pc->idle);
  }
  free_contexts(drop);
  return 0;
}

int ihip_prompt_cache_acquire(ihip_prompt_cache* pc, const int32_t* prompt, int64_t n, ihip_mctx** out)
{
  if (!pc || !out || (n > 0 && !prompt)) return fail(IHIP_E_ARG, "ihip_prompt_cache_acquire");
  *out = nullptr;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    int64_t best = -1, longest = 0;
    for (size_t i = 0; i < pc->idle.size(); i++) {
      // as Reuse keeps them: the last token is always computed again
      const int64_t common = usable(pc->idle[i], prompt, n - 1);
      if (common > longest) {
        longest = common;
        best = (int64_t)i;
      }
    }
    // no shared token: the buffers of the least recently used, once full
    if (best < 0 && !pc->idle.empty() && (int64_t)pc->idle.size() >= pc->slots) best = 0;
    if (best >= 0) {
      *out = pc->idle[best];
      pc->idle.erase(pc->idle.begin() + best);
      return 0;
    }
  }
  return ihip_model_new_context(pc->m, out);
}

int ihip_prompt_cache_release(ihip_prompt_cache* pc, ihip_mctx* s, int64_t reused)
{
  if (!pc) return fail(IHIP_E_ARG, "ihip_prompt_cache_release");
  if (!s) return 0;
  if (s->m != pc->m) return fail(IHIP_E_ARG, "ihip_prompt_cache_release: a context of another model");
  ihip_mctx* drop = nullptr;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    pc->requests++;
    if (reused > 0) {
      pc->hits++;
      pc->reused += reused;
    }
    if (pc->slots == 0) {
      drop = s;
    } else {
      if ((int64_t)pc->idle.size() >= pc->slots) {
        drop = pc->idle.front();
        pc->idle.erase(pc->idle.begin());
      }
      pc->idle.push_back(s);
    }
  }
  if (drop) ihip_context_destroy(drop);
  return 0;
}

int ihip_prompt_cache_stats(ihip_prompt_cache* pc, int64_t* requests, int64_t* hits, int64_t* reused,
                            int64_t* idle)
{
  if (!pc) return fail(IHIP_E_ARG, "ihip_prompt_cache_stats");
  std::lock_guard<std::mutex> g(pc->mu);
  if (requests) *requests = pc->requests;
  if (hits) *hits = pc->hits;
  if (reused) *reused = pc->reused;
  if (idle) *idle = (int64_t)pc->idle.size();
  return 0;
}

int ihip_model_use_graphs(ihip_model* m, int on)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_use_graphs");
  m->use_graphs = on != 0;
  return 0;
}

int ihip_model_check_route(ihip_model* m, int on)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_check_route");
  std::lock_guard<std::mutex> g(m->c->lock);
  m->check_route = on != 0;
  return 0;
}

int ihip_model_route_stats(ihip_model* m, int64_t* checks, int64_t* mismatches, double* max_diff)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_route_stats");
  std::lock_guard<std::mutex> g(m->c->lock);
  if (checks) *checks = m->route_checks;
  if (mismatches) *mismatches = m->route_mismatches;
  if (max_diff) *max_diff = m->route_max_diff;
  return 0;
}

int ihip_model_route_tape(ihip_model* m, const int32_t* ids, const float* weights, int64_t rows)
{
  if (!m || rows < 0 || (rows > 0 && (!ids || !weights))) return fail(IHIP_E_ARG, "ihip_model_route_tape");
  std::lock_guard<std::mutex> g(m->c->lock);
  const int64_t K = m->d.experts_used;
  if (rows > 0 && K < 1) return fail(IHIP_E_ARG, "ihip_model_route_tape: the model has no experts");
  for (int64_t i = 0; i < rows * K; i++)
    if (ids[i] < 0 || ids[i] >= m->d.experts) return fail(IHIP_E_ARG, "ihip_model_route_tape: an expert id out of range");
  m->tape_ids.assign(ids, ids + rows * K);
  m->tape_w.assign(weights, weights + rows * K);
  m->tape_rows = rows;
  m->tape_pos = m->tape_routes = m->tape_differs = 0;
  m->tape_gap = 0;
  return 0;
}

int ihip_model_debug_layer(ihip_model* m, int layer, float* rows)
{
  if (!m || (rows && (layer < -1 || layer >= m->d.layers))) return fail(IHIP_E_ARG, "ihip_model_debug_layer");
  m->dbg_host = rows;
  m->dbg_layer = layer;
  return 0;
}

int ihip_model_route_tape_stats(ihip_model* m, int64_t* routes, int64_t* differs, double* gap,
                                int64_t* pending)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_route_tape_stats");
  std::lock_guard<std::mutex> g(m->c->lock);
  if (routes) *routes = m->tape_routes;
  if (differs) *differs = m->tape_differs;
  if (gap) *gap = m->tape_gap;
  if (pending) *pending = m->tape_rows - m->tape_pos;
  return 0;
}

int ihip_model_timing(ihip_model* m, double* prefill_ms, double* decode_ms)
{
  if (!m) return fail(IHIP_E_ARG, "ihip_model_timing");
  if (prefill_ms) *prefill_ms = m->def->prefill_ms;
  if (decode_ms) *decode_ms = m->def->decode_ms;
  return 0;
}

}  // extern "C"
