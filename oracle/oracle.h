/* oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement in plain C of the reference's CPU arithmetic for the
 * quantized-inference hot path (landrix/mormot2-ai, Object Pascal), used as
 * the checker of the HIP backend. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Each function cites the reference file:line it follows (paths under
 * src/infer/ of the reference). The reference itself cannot be compiled here
 * (Object Pascal + mORMot2, no FPC/Delphi in the image), so oracle/_ref stays
 * empty; parity is pinned by the reference's golden vectors
 * (tests/data/infer-ref/{q8,q4,q5,q51,qk,mxfp4,ops}, copied as data into
 * tests/golden/) and by the closed-form checks of tests/test_oracle*.py.
 *
 * Pinning status per function (see the tests named):
 *   orc_half_to_single_bits, orc_single_to_half  - q8 half/x + half/bits vectors + all
 *       65536 half patterns against numpy's IEEE conversion
 *   orc_e8m0_half_bits                           - closed form 2^(e-128)
 *   orc_row_to_f32                               - q8/q4/q5/q51/qk/mxfp4 dequant/y
 *   orc_quantize_q8_0 (ties even / away)         - q8 quant/blocks, q4 q8ref/blocks
 *   orc_quantize_q4_0                            - q4 quant/blocks
 *   orc_quantize_q8_k                            - qk q8k/blocks
 *   orc_linear (Q8 arithmetic)                   - linear/y of every format
 *   orc_linear_f32                               - ops linear/y, brute force
 *   orc_rmsnorm, orc_swiglu, orc_rope            - closed forms in numpy (float64)
 *   orc_causal_attention                         - ops softmax/y + numpy float64
 *   orc_route                                    - brute-force numpy softmax/top-k
 *   orc_argmax                                   - numpy argmax + NaN/tie cases
 *   orc_rotary                                   - numpy float32 step replay
 *   orc_delta_prep, orc_delta_rule, orc_gate_sigmoid - transformers' float32
 *       intermediate states and logits of tiny-qwen35 (tests/test_qwen35.py)
 *   orc_rotary2, orc_geglu, orc_softcap           - transformers' float32 logits
 *       of tiny-gemma4 and closed forms (tests/test_gemma4.py)
 *   orc_model_*                                  - composed of the above;
 *       checked against a numpy float64 forward of a tiny model
 */
#ifndef ORACLE_H
#define ORACLE_H

#include <stdint.h>
#include "../include/mormot_ai_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* tensor.pas:296-326 InferHalfToSingleBits; :328-377 InferSingleToHalf */
uint32_t orc_half_to_single_bits(uint16_t h);
float orc_half_to_single(uint16_t h);
uint16_t orc_single_to_half(float f);
/* tensor.pas:459-465 InferE8M0HalfBits */
uint32_t orc_e8m0_half_bits(uint8_t e);
/* tensor.pas:187-192 INFER_DTYPE_SIZE / INFER_DTYPE_BLOCK */
int orc_block_size(int dtype);
int orc_block_values(int dtype);
/* tensor.pas:467-602 InferRowToF32: row `row` of [*, cols] */
int orc_row_to_f32(const void* data, int dtype, int64_t row, int64_t cols,
                   float* dst);

/* backend.cpu.pas:634-699 QuantizeQ8_0: returns 0, or 1 + index of the first
 * non-finite value */
int64_t orc_quantize_q8_0(const float* x, int64_t n, void* blocks, int ties_away);
/* backend.cpu.pas:703-756 InferQuantizeRowQ4_0 */
int64_t orc_quantize_q4_0(const float* x, int64_t n, void* blocks);
/* backend.cpu.pas:758-819 InferQuantizeRowQ8_K */
int64_t orc_quantize_q8_k(const float* x, int64_t n, void* blocks);

/* backend.cpu.pas:1472-1566 TInferCpuBackend.Linear: the quantized
 * arithmetic for block types, the double F32 sum for F32; BF16 widened to
 * F32 first (decoder.pas:2211-2221). threads > 1 splits the outputs, every
 * output keeps its own sequential sum: the same bits at any thread count */
int orc_linear(const float* x, int64_t rows, int64_t in, const void* w,
               int dtype, int64_t out, const float* bias, float* y, int threads);
/* the tier-2 oracle of test.infer.cuda.pas:815-831: F32 weights from
 * InferRowToF32, the double Linear of backend.cpu.pas:1548-1565 */
int orc_linear_f32(const float* x, int64_t rows, int64_t in, const void* w,
                   int dtype, int64_t out, const float* bias, float* y, int threads);

/* backend.cpu.pas:1769-1795 */
void orc_rmsnorm(const float* x, int64_t rows, int64_t cols, const float* w,
                 double eps, float* y);
/* backend.cpu.pas:1797-1834 */
void orc_swiglu(float* gate, const float* up, int64_t n, float alpha, float limit);
/* backend.cpu.pas:1862-1888 */
void orc_rope(float* x, int64_t rows, int64_t heads, int64_t head_dim,
              const float* cos_, const float* sin_, int64_t rot_dim);
/* backend.cpu.pas:1233-1380, the reference (double) branch of CausalRows */
void orc_causal_attention(const float* q, int64_t rows, int64_t heads,
                          int64_t head_dim, const float* keys, const float* values,
                          int64_t past, int64_t kv_heads, float* y, int64_t window,
                          const float* sinks, double scale);
/* the same, the heads split over `threads` OpenMP threads (bit-identical) */
void orc_causal_attention_mt(const float* q, int64_t rows, int64_t heads, int64_t d,
                             const float* keys, const float* values, int64_t past,
                             int64_t kvh, float* y, int64_t window, const float* sinks,
                             double scale, int threads);
/* decoder.pas:2901-2949 TDecoderModel.Route (no expert scale, no tape) */
void orc_route(const float* logits, int64_t experts, int64_t k, int norm_topk,
               int32_t* chosen, float* weights);
/* sampler.pas:123-160 InferArgMax */
int64_t orc_argmax(const float* v, int64_t n);

/* decoder.pas:2524-2537 Rotary2: the second rotary set over heads of hd2 */
int orc_rotary2(const ihip_model_desc* d, int64_t hd2, int64_t first, int64_t rows, float* cs);
/* backend.cpu.pas:1836-1860 GeluTanhGlu: gate := gelu_tanh(gate) * up */
void orc_geglu(float* gate, const float* up, int64_t n);
/* decoder.pas:1293-1312 InferSoftcap */
void orc_softcap(float* x, int64_t n, double cap);
/* deltanet.c: GateBySigmoid (decoder.pas:2594-2610): a[i] *= sigmoid(gate[i]) */
void orc_gate_sigmoid(float* a, const float* gate, int64_t n);
/* deltanet.c: TDecoderModel.DeltaPrep (decoder.pas:2755-2855) over every item
 * in order: qkv [rows, 2 kh dk + vh dv] convolved (conv [channels, kw - 1],
 * oldest first, moved on) and silu'd, q/k heads L2-normed (q times dk^-0.5);
 * beta = sigmoid, decay = exp(neg_a * softplus(decay + dt_bias)), z = silu(z) */
void orc_delta_prep(float* qkv, float* beta, float* decay, float* z, int64_t rows,
                    float* conv, const float* conv_w, const float* dt_bias, const float* neg_a,
                    int64_t kh, int64_t vh, int64_t dk, int64_t dv, int64_t kw);
/* deltanet.c: TInferCpuBackend.DeltaRule (backend.cpu.pas:1890-1972, double):
 * state [vh, dv, dk], y [rows, vh * dv]; value head h reads key head
 * (h / group) % kh */
void orc_delta_rule(const float* qkv, int64_t rows, int64_t stride, int64_t kh, int64_t vh,
                    int64_t dk, int64_t dv, int64_t group, const float* beta, const float* decay,
                    float* state, float* y);

/* decoder.pas:1735-1750 + 1759-1829: the inverse frequencies (and YaRN) of a
 * model; decoder.pas:2539-2561 Rotary: [rows, half] cos, then sin */
int orc_rotary(const ihip_model_desc* d, int64_t first, int64_t rows, float* cs);

/* the CPU decoder (decoder.pas:3245-3369 ForwardPart with TInferCpuBackend):
 * kv_f16 != 0 rounds every cached key/value to half (the device's F16 cache
 * restated, not a reference behaviour) */
typedef struct orc_model orc_model;
int orc_model_create(const ihip_model_desc* d, int64_t max_tokens, int kv_f16,
                     int threads, orc_model** out);
void orc_model_destroy(orc_model* m);
/* f32 != 0: every Linear in the F32 arithmetic (orc_linear_f32) instead of
 * the CPU's quantized one - the oracle of the device's IHIP_MODE_F32 */
void orc_model_set_f32(orc_model* m, int f32);
/* fast != 0: TInferCpuFastBackend's default mode (fast.c: AVX2 Linear on
 * tiles of 16 outputs over the pool, the fast attention) - the timed CPU
 * baseline; needs orc_fast_available() */
void orc_model_set_fast(orc_model* m, int fast);
/* the worker threads of the model's Linear and attention */
void orc_model_set_threads(orc_model* m, int threads);
/* ids, or embedding rows [count, hidden] in their place (ForwardEmbeds);
 * normed (or NULL): the last row after the final norm */
int orc_model_forward_rows(orc_model* m, const int32_t* ids, const float* embeds, int64_t count,
                           float* logits, int all_logits, float* normed);
/* back to length tokens (TDecoderContext.Truncate) */
int orc_model_truncate(orc_model* m, int64_t length);
/* the smallest k-th vs (k+1)-th router logit gap since the last call (then reset) */
double orc_model_route_gap(orc_model* m);
/* TDecoderRouteTape recording: the k picks (by id) and weights of every
 * routed row from now on appended to ids / w [cap][k] (NULL: off) */
void orc_model_route_record(orc_model* m, int32_t* ids, float* w, int64_t cap);
int64_t orc_model_route_recorded(orc_model* m);
/* a test hook: the residual rows after layer `layer` (-1: every layer, one after another) of each later forward copied to rows (NULL: off) */
void orc_model_debug_layer(orc_model* m, int64_t layer, float* rows);
int orc_model_forward(orc_model* m, const int32_t* ids, int64_t count,
                      float* logits, int all_logits);
/* decoder.pas:3390-3426 Greedy; margins[i] = top1 - top2 logit of step i */
int orc_model_greedy(orc_model* m, const int32_t* prompt, int64_t n,
                     int64_t max_new, int32_t* out_ids, float* margins);

/* sampler.c: TInferSampler (sampler.pas:52-435) */
double orc_splitmix_next(uint64_t* state);
int orc_sampler_create(double temperature, int32_t top_k, double top_p, double min_p,
                       int64_t seed, void** out);
void orc_sampler_destroy(void* s);
int64_t orc_sampler_next(void* s, const float* logits, int64_t count);

/* fast.c: TInferCpuFastBackend (backend.cpu.pas:1975-2506) with AVX2 */
int orc_fast_available(void);
int orc_fast_linear(const float* x, int64_t rows, int64_t in, const void* w, int dtype,
                    int64_t out, const float* bias, float* y, int threads);
void orc_fast_attention(const float* q, int64_t rows, int64_t heads, int64_t head_dim,
                        const float* keys, const float* values, int64_t past, int64_t kv_heads,
                        float* y, int64_t window, const float* sinks, int threads);

#ifdef __cplusplus
}
#endif

#endif
