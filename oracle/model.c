/* model.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * The CPU decoder: TDecoderModel.ForwardPart (decoder.pas:3245-3369) with
 * AttentionBlock (:2625-2702, the output gate and partial rotary of Qwen3.5
 * included), DeltaNetBlock (:2704-2753), DenseBlock/DenseFfn (:2866-2899),
 * MoeBlock (:3037-3053) and Experts (:3092-3150) over TInferCpuBackend, and
 * Greedy (:3390-3426). */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

struct orc_model {
  ihip_model_desc d;
  ihip_layer_desc* layer;
  int64_t max_tokens, length;
  int kv_f16, threads, f32, fast;
  /* the smallest gap between the k-th and (k+1)-th router logit of any
   * routed row since the last orc_model_route_gap (a near tie there could
   * pick another expert on another arithmetic) */
  double route_gap;
  /* TDecoderRouteTape in drmRecord (decoder.pas:2955-2990): every routed
   * row's k picks (by id) and weights appended here, up to rec_cap rows */
  int32_t* rec_ids;
  float* rec_w;
  int64_t rec_cap, rec_rows;
  float** keys;
  float** values;
  /* per DeltaNet layer: the last conv - 1 inputs of every channel and the
   * state S [value heads, value dim, key dim] (TDecoderContext.fConv/fState) */
  float** conv;
  float** state;
  int recurrent;
  /* a test's capture of the residual rows after layer dbg_layer */
  float* dbg;
  int64_t dbg_layer;
};

static uint64_t row_bytes(int t, int64_t cols)
{
  return (uint64_t)(cols / orc_block_values(t)) * orc_block_size(t);
}

int orc_model_create(const ihip_model_desc* d, int64_t max_tokens, int kv_f16, int threads,
                     orc_model** out)
{
  orc_model* m = (orc_model*)calloc(1, sizeof(*m));
  m->d = *d;
  m->layer = (ihip_layer_desc*)malloc(d->layers * sizeof(ihip_layer_desc));
  memcpy(m->layer, d->layer, d->layers * sizeof(ihip_layer_desc));
  m->max_tokens = max_tokens;
  m->kv_f16 = kv_f16;
  m->threads = threads > 0 ? threads : 1;
  m->route_gap = INFINITY;
  m->keys = (float**)calloc(d->layers, sizeof(float*));
  m->values = (float**)calloc(d->layers, sizeof(float*));
  m->conv = (float**)calloc(d->layers, sizeof(float*));
  m->state = (float**)calloc(d->layers, sizeof(float*));
  const int64_t cd = 2 * (int64_t)d->lin_key_heads * d->lin_key_dim +
                     (int64_t)d->lin_value_heads * d->lin_value_dim;
  for (int l = 0; l < d->layers; l++) {
    if (d->layer[l].mixer == IHIP_MIXER_DELTANET) {
      m->recurrent = 1;
      m->conv[l] = (float*)calloc(cd * (d->lin_conv > 1 ? d->lin_conv - 1 : 1), sizeof(float));
      m->state[l] = (float*)calloc((int64_t)d->lin_value_heads * d->lin_value_dim * d->lin_key_dim,
                                   sizeof(float));
      continue;
    }
    const ihip_layer_desc* L = &d->layer[l];
    const int64_t lkvw = (int64_t)(L->kv_heads > 0 ? L->kv_heads : d->kv_heads) *
                         (L->head_dim > 0 ? L->head_dim : d->head_dim);
    m->keys[l] = (float*)calloc(max_tokens * lkvw, sizeof(float));
    m->values[l] = (float*)calloc(max_tokens * lkvw, sizeof(float));
  }
  *out = m;
  return 0;
}

void orc_model_set_f32(orc_model* m, int f32) { m->f32 = f32; }

void orc_model_set_threads(orc_model* m, int threads) { m->threads = threads > 0 ? threads : 1; }

void orc_model_set_fast(orc_model* m, int fast) { m->fast = fast && orc_fast_available(); }

int orc_model_truncate(orc_model* m, int64_t length)
{
  if (length < 0 || length > m->length) return IHIP_E_ARG;
  /* a recurrent state holds the whole sequence: back to 0 only
   * (TDecoderContext.Restorable, decoder.pas:1180-1197, without restore
   * points) */
  if (m->recurrent && length != 0 && length != m->length) return IHIP_E_ARG;
  m->length = length;
  return 0;
}

void orc_model_route_record(orc_model* m, int32_t* ids, float* w, int64_t cap)
{
  m->rec_ids = ids;
  m->rec_w = w;
  m->rec_cap = ids && w ? cap : 0;
  m->rec_rows = 0;
}

int64_t orc_model_route_recorded(orc_model* m) { return m->rec_rows; }

void orc_model_debug_layer(orc_model* m, int64_t layer, float* rows)
{
  m->dbg = rows;
  m->dbg_layer = layer;
}

double orc_model_route_gap(orc_model* m)
{
  double g = m->route_gap;
  m->route_gap = INFINITY;
  return g;
}

/* logit of the k-th pick minus the largest logit not picked */
static double route_gap(const float* lg, int64_t e, const int32_t* chosen, int64_t k)
{
  double kth = INFINITY, next = -INFINITY;
  for (int64_t j = 0; j < k; j++)
    if (lg[chosen[j]] < kth) kth = lg[chosen[j]];
  for (int64_t i = 0; i < e; i++) {
    int taken = 0;
    for (int64_t j = 0; j < k; j++)
      if (chosen[j] == i) taken = 1;
    if (!taken && lg[i] > next) next = lg[i];
  }
  return kth - next;
}

void orc_model_destroy(orc_model* m)
{
  if (!m) return;
  for (int l = 0; l < m->d.layers; l++) {
    free(m->keys[l]);
    free(m->values[l]);
    free(m->conv[l]);
    free(m->state[l]);
  }
  free(m->keys);
  free(m->values);
  free(m->conv);
  free(m->state);
  free(m->layer);
  free(m);
}

static int lin(orc_model* m, const float* x, int64_t rows, int64_t in, ihip_tensor w,
               uint64_t offset, int64_t out, const float* bias, float* y)
{
  if (m->fast)
    return orc_fast_linear(x, rows, in, (const uint8_t*)w.data + offset, w.dtype, out, bias, y,
                           m->threads);
  if (m->f32)
    return orc_linear_f32(x, rows, in, (const uint8_t*)w.data + offset, w.dtype, out, bias, y,
                          m->threads);
  return orc_linear(x, rows, in, (const uint8_t*)w.data + offset, w.dtype, out, bias, y,
                    m->threads);
}

static void add(float* x, const float* t, int64_t n)
{
  for (int64_t i = 0; i < n; i++) x[i] = x[i] + t[i];
}

/* TDecoderModel.Activate (decoder.pas:2857-2863): SwiGLU or GeGLU */
static void activate(const ihip_model_desc* d, float* gate, const float* up, int64_t n)
{
  if (d->activation == IHIP_ACT_GELU_TANH)
    orc_geglu(gate, up, n);
  else
    orc_swiglu(gate, up, n, d->swiglu_alpha, d->swiglu_limit);
}

static float half_round(float v)
{
  return orc_half_to_single(orc_single_to_half(v));
}

/* ForwardRows (TQwen3Model.Forward / ForwardEmbeds): ids, or embedding rows
 * [n, hidden] in their place; normed (or NULL): the last row after the final
 * norm */
int orc_model_forward_rows(orc_model* m, const int32_t* ids, const float* embeds, int64_t n,
                           float* logits, int all_logits, float* normed);

int orc_model_forward(orc_model* m, const int32_t* ids, int64_t n, float* logits,
                      int all_logits)
{
  return orc_model_forward_rows(m, ids, NULL, n, logits, all_logits, NULL);
}

int orc_model_forward_rows(orc_model* m, const int32_t* ids, const float* embeds, int64_t n,
                           float* logits, int all_logits, float* normed)
{
  const ihip_model_desc* d = &m->d;
  const int64_t h = d->hidden, past = m->length;
  const int64_t rot = d->rope_dims > 0 ? d->rope_dims : d->head_dim, half = rot / 2;
  /* the widest heads of any layer (Gemma 4: per layer), and the heads of the
   * second rotary set */
  int64_t qw = (int64_t)d->heads * d->head_dim, kvw = (int64_t)d->kv_heads * d->head_dim,
          hdmax = d->head_dim, hd2 = 0;
  for (int l = 0; l < d->layers; l++) {
    const ihip_layer_desc* L = &m->layer[l];
    const int64_t lhd = L->head_dim > 0 ? L->head_dim : d->head_dim;
    const int64_t lkvh = L->kv_heads > 0 ? L->kv_heads : d->kv_heads;
    if (d->heads * lhd > qw) qw = d->heads * lhd;
    if (lkvh * lhd > kvw) kvw = lkvh * lhd;
    if (lhd > hdmax) hdmax = lhd;
    if (L->rope_set) hd2 = lhd;
  }
  const int64_t kh = d->lin_key_heads, vh = d->lin_value_heads, dk = d->lin_key_dim,
                dv = d->lin_value_dim, vd = vh * dv, cd = 2 * kh * dk + vd;
  /* LinGroup (decoder.pas:2457-2463) */
  const int64_t group = (d->lin_tiled || kh <= 0) ? 1 : vh / kh;
  int64_t f = d->ffn > d->expert_ffn ? d->ffn : d->expert_ffn;
  int err = 0;
  if (n <= 0 || past + n > m->max_tokens || (!ids && !embeds))
    return IHIP_E_ARG;
  if (ids)
    for (int64_t i = 0; i < n; i++)
      if (ids[i] < 0 || ids[i] >= d->vocab) return IHIP_E_ARG;
  float* x = (float*)malloc(n * h * 4);
  float* hh = (float*)malloc(n * h * 4);
  float* tmp = (float*)malloc(n * h * 4);
  float* q = (float*)malloc(n * qw * 4);
  float* k = (float*)malloc(n * kvw * 4);
  float* v = (float*)malloc(n * kvw * 4);
  float* attn = (float*)malloc(n * qw * 4);
  float* gate = (float*)malloc(n * (f > 0 ? f : 1) * 4);
  float* up = (float*)malloc(n * (f > 0 ? f : 1) * 4);
  float* cs = (float*)malloc(n * hdmax * 4);
  float* cs2 = (float*)malloc(n * (hd2 > 0 ? hd2 : 1) * 4);
  float* ones = (float*)malloc(hdmax * 4);
  float* dense = (float*)malloc(n * h * 4);
  for (int64_t i = 0; i < hdmax; i++) ones[i] = 1.0f;
  int64_t E = d->experts > 0 ? d->experts : 1, K = d->experts_used > 0 ? d->experts_used : 1;
  float* route = (float*)malloc(n * E * 4);
  int32_t* chosen = (int32_t*)malloc(n * K * 4);
  float* cw = (float*)malloc(n * K * 4);
  float* gather = (float*)malloc(n * h * 4);
  float* eout = (float*)malloc(n * h * 4);
  int64_t* rowi = (int64_t*)malloc(n * sizeof(int64_t));
  float* roww = (float*)malloc(n * 4);
  float* qg = (float*)malloc(n * 2 * qw * 4);
  float* gq = (float*)malloc(n * qw * 4);
  float* qkv = (float*)malloc(n * (cd > 0 ? cd : 1) * 4);
  float* z = (float*)malloc(n * (vd > 0 ? vd : 1) * 4);
  float* beta = (float*)malloc(n * (vh > 0 ? vh : 1) * 4);
  float* decay = (float*)malloc(n * (vh > 0 ? vh : 1) * 4);
  float* core = (float*)malloc(n * (vd > 0 ? vd : 1) * 4);

  orc_rotary(d, past, n, cs);
  if (hd2 > 0) orc_rotary2(d, hd2, past, n, cs2);
  if (ids) {
    for (int64_t i = 0; i < n; i++)
      orc_row_to_f32(d->embed.data, d->embed.dtype, ids[i], h, x + i * h);
    /* Gemma scales the embeddings of ids (ForwardPart, decoder.pas:3305-3309) */
    if (d->embed_scale > 0)
      for (int64_t i = 0; i < n * h; i++) x[i] = x[i] * d->embed_scale;
  } else {
    memcpy(x, embeds, n * h * 4);
  }
  for (int l = 0; l < d->layers && !err; l++) {
    const ihip_layer_desc* L = &m->layer[l];
    if (L->mixer == IHIP_MIXER_DELTANET) {
      /* DeltaNetBlock: pre-norm, the four projections, DeltaPrep, the
       * recurrence, the gated RMSNorm per value head, the output projection */
      orc_rmsnorm(x, n, h, (const float*)L->input_norm.data, d->rms_eps, hh);
      err |= lin(m, hh, n, h, L->lin_qkv, 0, cd, NULL, qkv);
      err |= lin(m, hh, n, h, L->lin_z, 0, vd, NULL, z);
      err |= lin(m, hh, n, h, L->lin_b, 0, vh, NULL, beta);
      err |= lin(m, hh, n, h, L->lin_a, 0, vh, NULL, decay);
      if (past == 0) {
        memset(m->conv[l], 0, cd * (d->lin_conv > 1 ? d->lin_conv - 1 : 1) * 4);
        memset(m->state[l], 0, vh * dv * dk * 4);
      }
      orc_delta_prep(qkv, beta, decay, z, n, m->conv[l], (const float*)L->lin_conv.data,
                     (const float*)L->lin_dt_bias.data, (const float*)L->lin_neg_a.data, kh, vh,
                     dk, dv, d->lin_conv);
      orc_delta_rule(qkv, n, cd, kh, vh, dk, dv, group, beta, decay, m->state[l], core);
      orc_rmsnorm(core, n * vh, dv, (const float*)L->lin_norm.data, d->rms_eps, core);
      for (int64_t i = 0; i < n * vd; i++) core[i] = core[i] * z[i];
      err |= lin(m, core, n, vd, L->lin_out, 0, h, NULL, tmp);
      add(x, tmp, n * h);
      goto ffn;
    }
    /* AttentionBlock, with this layer's heads */
    const int64_t hd = L->head_dim > 0 ? L->head_dim : d->head_dim;
    const int64_t kvh = L->kv_heads > 0 ? L->kv_heads : d->kv_heads;
    const int64_t qw = (int64_t)d->heads * hd, kvw = kvh * hd;
    orc_rmsnorm(x, n, h, (const float*)L->input_norm.data, d->rms_eps, hh);
    if (L->output_gate) {
      /* per head the query, then its gate */
      err |= lin(m, hh, n, h, L->q, 0, 2 * qw, NULL, qg);
      for (int64_t r = 0; r < n * d->heads; r++) {
        memcpy(q + r * hd, qg + r * 2 * hd, hd * 4);
        memcpy(gq + r * hd, qg + r * 2 * hd + hd, hd * 4);
      }
    } else {
      err |= lin(m, hh, n, h, L->q, 0, qw, (const float*)L->q_bias.data, q);
    }
    err |= lin(m, hh, n, h, L->k, 0, kvw, (const float*)L->k_bias.data, k);
    if (L->k_is_v)
      memcpy(v, k, n * kvw * 4);  /* the values are the raw keys */
    else
      err |= lin(m, hh, n, h, L->v, 0, kvw, (const float*)L->v_bias.data, v);
    if (L->q_norm.data) {
      orc_rmsnorm(q, n * d->heads, hd, (const float*)L->q_norm.data, d->rms_eps, q);
      orc_rmsnorm(k, n * kvh, hd, (const float*)L->k_norm.data, d->rms_eps, k);
    }
    if (d->value_norm) orc_rmsnorm(v, n * kvh, hd, ones, d->rms_eps, v);
    if (L->no_rope) {
      /* a NoPE layer (decoder.pas:139, NoRope): q and k as they are */
    } else if (L->rope_set) {
      /* the second set: every pair of the head, frequency 0 beyond its share */
      orc_rope(q, n, d->heads, hd, cs2, cs2 + n * (hd / 2), 0);
      orc_rope(k, n, kvh, hd, cs2, cs2 + n * (hd / 2), 0);
    } else {
      orc_rope(q, n, d->heads, hd, cs, cs + n * half, rot);
      orc_rope(k, n, kvh, hd, cs, cs + n * half, rot);
    }
    float* kc = m->keys[l] + past * kvw;
    float* vc = m->values[l] + past * kvw;
    for (int64_t i = 0; i < n * kvw; i++) {
      kc[i] = m->kv_f16 ? half_round(k[i]) : k[i];
      vc[i] = m->kv_f16 ? half_round(v[i]) : v[i];
    }
    if (m->fast)
      orc_fast_attention(q, n, d->heads, hd, m->keys[l], m->values[l], past, kvh, attn,
                         L->window, (const float*)L->sinks.data, m->threads);
    else
      orc_causal_attention_mt(q, n, d->heads, hd, m->keys[l], m->values[l], past, kvh,
                              attn, L->window, (const float*)L->sinks.data, d->attention_scale,
                              m->threads);
    if (L->output_gate) orc_gate_sigmoid(attn, gq, n * qw);
    err |= lin(m, attn, n, qw, L->o, 0, h, (const float*)L->o_bias.data, tmp);
    /* Gemma: the attention output normed before the residual */
    if (L->attn_out_norm.data)
      orc_rmsnorm(tmp, n, h, (const float*)L->attn_out_norm.data, d->rms_eps, tmp);
    add(x, tmp, n * h);
  ffn:
    /* the feed-forward block: DenseBlock, MoeBlock or DenseMoeBlock
     * (decoder.pas:2880-2899, :3037-3091), then Gemma's layer scalar */
    orc_rmsnorm(x, n, h, (const float*)L->post_norm.data, d->rms_eps, hh);
    if (L->moe != IHIP_FFN_MOE) {
      err |= lin(m, hh, n, h, L->gate, 0, d->ffn, NULL, gate);
      err |= lin(m, hh, n, h, L->up, 0, d->ffn, NULL, up);
      activate(d, gate, up, n * d->ffn);
      err |= lin(m, gate, n, d->ffn, L->down, 0, h, NULL, tmp);
    }
    if (L->moe != IHIP_FFN_DENSE) {
      float* dst = tmp;
      if (L->moe == IHIP_FFN_DENSE_MOE) {
        /* the dense output normed; the router on the residual's own norm, the
         * experts on another, their sum normed */
        orc_rmsnorm(tmp, n, h, (const float*)L->dense_out_norm.data, d->rms_eps, tmp);
        orc_rmsnorm(x, n, h, (const float*)L->router_norm.data, d->rms_eps, hh);
        err |= lin(m, hh, n, h, L->router, 0, E, NULL, route);
        orc_rmsnorm(x, n, h, (const float*)L->moe_in_norm.data, d->rms_eps, hh);
        dst = dense;
      } else {
        err |= lin(m, hh, n, h, L->router, 0, E, (const float*)L->router_bias.data, route);
      }
      /* Experts (decoder.pas:3092-3150): the route of every row, then
       * expert by expert in id order over its gathered rows */
      const int64_t fi = d->expert_ffn;
      const float* escale = (const float*)L->expert_scale.data;
      for (int64_t r = 0; r < n; r++) {
        orc_route(route + r * E, E, K, d->norm_topk, chosen + r * K, cw + r * K);
        if (K < E) {
          double g = route_gap(route + r * E, E, chosen + r * K, K);
          if (g < m->route_gap) m->route_gap = g;
        }
        if (escale)
          for (int64_t j = 0; j < K; j++) cw[r * K + j] = cw[r * K + j] * escale[chosen[r * K + j]];
        if (m->rec_rows < m->rec_cap) {
          memcpy(m->rec_ids + m->rec_rows * K, chosen + r * K, K * 4);
          memcpy(m->rec_w + m->rec_rows * K, cw + r * K, K * 4);
          m->rec_rows++;
        }
      }
      memset(dst, 0, n * h * 4);
      /* gate and up of an expert: two tensors, or one [E, 2 fi, h] with the
       * gate rows first */
      const uint64_t rb = row_bytes(L->exp_gate.dtype, h);
      const uint64_t gstride = rb * fi * (L->exp_gate_up ? 2 : 1);
      const ihip_tensor ut = L->exp_gate_up ? L->exp_gate : L->exp_up;
      const uint64_t uoff = L->exp_gate_up ? rb * fi : 0;
      const uint64_t db = row_bytes(L->exp_down.dtype, fi) * h;
      for (int64_t e = 0; e < E; e++) {
        int64_t cnt = 0;
        for (int64_t r = 0; r < n; r++)
          for (int64_t j = 0; j < K; j++)
            if (chosen[r * K + j] == e) {
              rowi[cnt] = r;
              roww[cnt] = cw[r * K + j];
              memcpy(gather + cnt * h, hh + r * h, h * 4);
              cnt++;
            }
        if (cnt == 0) continue;
        const float* bg = L->exp_gate_bias.data ? (const float*)L->exp_gate_bias.data + e * fi : NULL;
        const float* bu = L->exp_up_bias.data ? (const float*)L->exp_up_bias.data + e * fi : NULL;
        const float* bd = L->exp_down_bias.data ? (const float*)L->exp_down_bias.data + e * h : NULL;
        err |= lin(m, gather, cnt, h, L->exp_gate, e * gstride, fi, bg, gate);
        err |= lin(m, gather, cnt, h, ut, e * gstride + uoff, fi, bu, up);
        activate(d, gate, up, cnt * fi);
        err |= lin(m, gate, cnt, fi, L->exp_down, e * db, h, bd, eout);
        for (int64_t c = 0; c < cnt; c++) {
          float w = roww[c];
          float* o = dst + rowi[c] * h;
          const float* src = eout + c * h;
          for (int64_t i = 0; i < h; i++) {
            float p = w * src[i];
            o[i] = o[i] + p;
          }
        }
      }
      if (L->moe == IHIP_FFN_DENSE_MOE) {
        orc_rmsnorm(dense, n, h, (const float*)L->moe_out_norm.data, d->rms_eps, dense);
        add(tmp, dense, n * h);
      }
    }
    /* Gemma: the feed-forward output normed before the residual */
    if (L->ffn_out_norm.data)
      orc_rmsnorm(tmp, n, h, (const float*)L->ffn_out_norm.data, d->rms_eps, tmp);
    add(x, tmp, n * h);
    /* Gemma: the whole state times the layer's scalar */
    if (L->scalar.data) {
      const float sc = *(const float*)L->scalar.data;
      for (int64_t i = 0; i < n * h; i++) x[i] = x[i] * sc;
    }
    if (m->dbg && (m->dbg_layer < 0 || l == m->dbg_layer))
      memcpy(m->dbg + (m->dbg_layer < 0 ? (size_t)l * n * h : 0), x, (size_t)(n * h) * 4);
  }
  if (!err) {
    m->length = past + n;
    if (logits || normed) {
      orc_rmsnorm(x, n, h, (const float*)d->final_norm.data, d->rms_eps, hh);
      if (normed) memcpy(normed, hh + (n - 1) * h, h * 4);
    }
    if (logits) {
      ihip_tensor head = d->head.data ? d->head : d->embed;
      if (all_logits)
        err |= lin(m, hh, n, h, head, 0, d->vocab, NULL, logits);
      else
        err |= lin(m, hh + (n - 1) * h, 1, h, head, 0, d->vocab, NULL, logits);
      if (d->logit_softcap > 0)
        orc_softcap(logits, (all_logits ? n : 1) * d->vocab, d->logit_softcap);
    }
  }
  free(x); free(hh); free(tmp); free(q); free(k); free(v); free(attn);
  free(gate); free(up); free(cs); free(route); free(chosen); free(cw);
  free(gather); free(eout); free(rowi); free(roww);
  free(qg); free(gq); free(qkv); free(z); free(beta); free(decay); free(core);
  free(cs2); free(ones); free(dense);
  return err ? IHIP_E_ARG : 0;
}

static float margin(const float* lg, int64_t n, int64_t best)
{
  float second = -INFINITY;
  for (int64_t i = 0; i < n; i++)
    if (i != best && lg[i] > second) second = lg[i];
  return lg[best] - second;
}

int orc_model_greedy(orc_model* m, const int32_t* prompt, int64_t n, int64_t max_new,
                     int32_t* out_ids, float* margins)
{
  int64_t V = m->d.vocab;
  float* lg = (float*)malloc(V * 4);
  int err = orc_model_forward(m, prompt, n, lg, 0);
  for (int64_t i = 0; i < max_new && !err; i++) {
    int64_t next = orc_argmax(lg, V);
    out_ids[i] = (int32_t)next;
    if (margins) margins[i] = margin(lg, V, next);
    int32_t id = (int32_t)next;
    if (i + 1 < max_new)
      err = orc_model_forward(m, &id, 1, lg, 0);
    else
      err = orc_model_forward(m, &id, 1, NULL, 0);
  }
  free(lg);
  return err;
}
