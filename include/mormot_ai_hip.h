/* mormot_ai_hip.h - the C-ABI of mormot.ai.infer.hip, the MI355X (gfx950)
 * quantized-inference backend of the mormot2-ai native engine.
 *
 * Every entry point takes plain pointers, sizes and integers: no C++ or torch
 * types cross this boundary. A Pascal unit binds them as `external` functions
 * of libmormot_ai_hip.so (cdecl); ctypes binds them the same way.
 *
 * Conventions
 * - status: every function returns 0 on success, else a negative IHIP_E_*
 *   code or a positive hipError_t; ihip_last_error() gives the text of the
 *   last failure of the calling thread (the EInferCuda message of
 *   src/infer/mormot.ai.infer.cuda.pas:475-487).
 * - device addresses are uint64_t (TCuDevicePtr of cuda.pas:137-175).
 * - dtype codes are the ordinals of TInferDType
 *   (src/infer/mormot.ai.infer.tensor.pas:47-62): the Pascal caller passes
 *   ord(w.DType) unchanged.
 * - one ihip_ctx is one device + one non-blocking stream; it may be used from
 *   any thread, one at a time (cuda.pas:13-15): callers serialise, as
 *   TInferCudaBackend.GpuLock does (backend.cuda.pas:102-104).
 */
#ifndef MORMOT_AI_HIP_H
#define MORMOT_AI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element and block types: TInferDType (tensor.pas:47-62) ---- */
enum {
  IHIP_F32 = 1,
  IHIP_F16 = 2,
  IHIP_BF16 = 3,
  IHIP_Q8_0 = 8,
  IHIP_Q4_0 = 9,
  IHIP_Q4_K = 10,
  IHIP_Q6_K = 11,
  IHIP_Q5_0 = 12,
  IHIP_MXFP4 = 13,
  IHIP_Q5_1 = 14
};

/* ---- arithmetic of a Linear ----
 * IHIP_MODE_F32: y = dequant(W) x in float, x in F32 - the contract of the
 *   reference's GPU kernels (tools/cuda/linear.cu:1-6): within 1e-5 of the
 *   double F32 Linear over InferRowToF32 weights.
 * IHIP_MODE_Q8: the arithmetic of TInferCpuBackend.Linear
 *   (src/infer/mormot.ai.infer.backend.cpu.pas:1409-1566): x quantized per row
 *   to Q8_0 (32-value block types) or Q8_K (Q4_K/Q6_K), exact integer block
 *   sums, the scales applied and summed in double; F32/BF16 weights summed in
 *   double. Same bits as the CPU up to the order of a double sum. */
enum { IHIP_MODE_F32 = 0, IHIP_MODE_Q8 = 1 };
/* or'ed into IHIP_MODE_Q8: x is a buffer already quantized by
 * ihip_enqueue_quantize (the quantization of a row shared by several
 * Linears is then done once) */
enum { IHIP_MODE_XQ = 2 };

/* ---- status codes ---- */
enum {
  IHIP_OK = 0,
  IHIP_E_ARG = -1,         /* an argument out of range (EInferCuda misuse) */
  IHIP_E_NODEVICE = -2,    /* no HIP device / library */
  IHIP_E_UNSUPPORTED = -3, /* this dtype/shape has no kernel: CPU fallback */
  IHIP_E_NONFINITE = -4,   /* a NaN/Inf activation where Q8 refuses it */
  IHIP_E_CAPTURE = -5,     /* not allowed while capturing, or capture misuse */
  IHIP_E_NOMEM = -6,       /* a fixed maximum size exceeded */
  IHIP_E_FORMAT = -7       /* a damaged, hostile or unsupported file (EInferError) */
};

typedef struct ihip_ctx ihip_ctx;
typedef struct ihip_model ihip_model;

/* ======================================================================
 * TInferCuda (src/infer/mormot.ai.infer.cuda.pas:179-254): device, stream,
 * buffers, graphs
 * ==================================================================== */

/* number of usable gfx950 devices, 0 when none (TInferCuda.Available,
 * cuda.pas:599-612) */
int ihip_available(void);
/* text of the last failure on this thread */
const char* ihip_last_error(void);
/* a context on device aDevice: loads the embedded gfx950 code object with
 * hipModuleLoadData (TInferCuda.Create, cuda.pas:494-573) */
int ihip_create(int device, ihip_ctx** out);
void ihip_destroy(ihip_ctx* ctx);
/* device name and total memory (cuda.pas:61-132 device queries) */
int ihip_device_info(ihip_ctx* ctx, char* name, int name_len,
                     uint64_t* total_mem, int* cus);

/* device buffers (TInferCuBuffer, cuda.pas:137-175) */
int ihip_alloc(ihip_ctx* ctx, uint64_t bytes, uint64_t* dev);
int ihip_free(ihip_ctx* ctx, uint64_t dev);
/* synchronous copies on the context's stream (Upload/Download) */
int ihip_upload(ihip_ctx* ctx, uint64_t dev, const void* host, uint64_t bytes);
int ihip_download(ihip_ctx* ctx, void* host, uint64_t dev, uint64_t bytes);
/* enqueued copies (cuMemcpyHtoDAsync / DtoD, cuda.pas:614-673); the host
 * memory must stay valid until the next synchronize */
int ihip_upload_async(ihip_ctx* ctx, uint64_t dev, const void* host, uint64_t bytes);
int ihip_copy_async(ihip_ctx* ctx, uint64_t dst, uint64_t src, uint64_t bytes);
int ihip_synchronize(ihip_ctx* ctx);

/* stream capture into a graph, instantiate or update, launch
 * (TInferCuda.CaptureBegin/CaptureEnd/GraphLaunch, cuda.pas:675-771) */
int ihip_capture_begin(ihip_ctx* ctx);
int ihip_capture_end(ihip_ctx* ctx, int slot);
int ihip_graph_launch(ihip_ctx* ctx, int slot);

/* elapsed milliseconds between two points of the stream, measured with HIP
 * events on that stream: ihip_event_record(ctx, i) marks point i (0..63) */
int ihip_event_record(ihip_ctx* ctx, int index);
int ihip_event_elapsed(ihip_ctx* ctx, int from, int to, float* ms);
/* the kernel timer (measurement; no counterpart in the reference, whose
 * benchmarks time whole passes): every later direct launch (not under
 * capture) of a kernel whose name starts with `prefix` is timed by the
 * start and end of its own dispatch, the durations a profiler reports;
 * NULL or "" stops it; at most `capacity` launches between two reads.
 * _read waits for the stream, returns the launches timed and their total
 * milliseconds since the last read, and starts over. */
int ihip_kernel_timer(ihip_ctx* ctx, const char* prefix, int64_t capacity);
int ihip_kernel_timer_read(ihip_ctx* ctx, int64_t* launches, double* total_ms);
/* the same, per kernel name (prefix "*" times every kernel): one line
 * "name launches total_ms" per kernel, in first-launch order, into text */
int ihip_kernel_timer_report(ihip_ctx* ctx, char* text, int64_t len);
/* a timing build (IHIP_TRACE) records phase clocks (100 MHz) of instrumented
 * kernels: launch k (k < count) of a kernel named prefix* into dev + k *
 * stride ([blocks][8] uint64); dev 0 stops; ignored by other builds */
int ihip_trace_buffer(ihip_ctx* ctx, uint64_t dev, uint64_t stride, int64_t count,
                      const char* prefix);

/* ======================================================================
 * TInferCudaBackend (src/infer/mormot.ai.infer.backend.cuda.pas:51-148)
 * ==================================================================== */

/* bytes of aCount values of aType (InferTypeBytes, tensor.pas:280-294); 0 if
 * aCount is no whole number of blocks */
uint64_t ihip_type_bytes(int dtype, uint64_t count);

/* the device copy of a weight, uploaded on first use and found again by
 * (host address, dtype, bytes) (TInferCudaBackend.Weight, backend.cuda.pas:
 * 414-449). The host data is [count, out, in] of dtype in GGUF layout; the
 * device copy is repacked per matrix into the HIP layout (quants, then
 * scales), of the same byte size: matrix m starts at dev + m * out * rowbytes,
 * as in the host tensor. count > 1: the experts of a layer. */
int ihip_weight(ihip_ctx* ctx, const void* host, int dtype, int64_t out,
                int64_t in, int64_t count, uint64_t* dev);
/* the repack of ihip_weight on the host: [count, out, in] GGUF blocks into
 * the HIP layout (inverse = 0), or back (inverse = 1); no device needed */
int ihip_repack(const void* src, void* dst, int dtype, int64_t out, int64_t in,
                int64_t count, int inverse);
/* F32 side data (biases, norms) kept by host address, as Weight(.., idtF32) */
int ihip_weight_f32(ihip_ctx* ctx, const float* host, int64_t count, uint64_t* dev);
/* drop the device copy of every weight overlapping [from, to)
 * (ForgetWeights, backend.cuda.pas:282-314); returns the new WeightEpoch */
int ihip_forget_weights(ihip_ctx* ctx, const void* from, const void* to);
int ihip_clear_weights(ihip_ctx* ctx);
/* true when Linear of aType with aIn inputs runs on the device
 * (GpuLinear, backend.cuda.pas:316-320) */
int ihip_gpu_linear(int dtype, int64_t in);

/* y[rows, out] = x[rows, in] * W^T + bias: W repacked at device address w
 * (EnqueueLinearAt, backend.cuda.pas:354-379); bias a device address of
 * [out] floats or 0; mode IHIP_MODE_F32 or IHIP_MODE_Q8; enqueued, no wait */
int ihip_enqueue_linear_at(ihip_ctx* ctx, uint64_t x, int64_t rows, int64_t in,
                           int dtype, uint64_t w, int64_t out, uint64_t y,
                           uint64_t bias, int mode);
/* ihip_enqueue_linear_at without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * Q8 quantized activations of a multi-row call go to a fixed device array of
 * IHIP_STATIC_SCRATCH_BYTES per GPU instead of the context's growable
 * scratch: rows * (in + in / 8) must fit (else IHIP_E_NOMEM, nothing
 * enqueued). Every call on one GPU shares that array; one context's stream
 * orders its own calls, so the first context to make a multi-row call holds
 * the array until it is destroyed and a multi-row call of another context on
 * that GPU is refused (IHIP_E_ARG, nothing enqueued). One-row calls use no
 * array. Same arguments and results as ihip_enqueue_linear_at. */
#define IHIP_STATIC_SCRATCH_BYTES (8u << 20)
int ihip_enqueue_linear_at_static(ihip_ctx* ctx, uint64_t x, int64_t rows, int64_t in,
                                  int dtype, uint64_t w, int64_t out, uint64_t y,
                                  uint64_t bias, int mode);
/* one token row through `slots` experts chosen on the device
 * (EnqueueLinearIds, backend.cuda.pas:386-412): slot s reads expert ids[s]
 * (int32 at a device address), its matrix at w + ids[s] * stride bytes
 * (stride = out * rowbytes), x row s / x_per_slot (x_per_slot = 1: row s,
 * k: the token of slot s when every token has k slots; 0: row 0), y row s;
 * bias: device [experts, out] floats (row ids[s]) or 0 */
int ihip_enqueue_linear_ids(ihip_ctx* ctx, uint64_t x, int64_t in, int dtype,
                            uint64_t w, int64_t stride, int64_t out,
                            uint64_t ids, int64_t slots, int x_per_slot,
                            uint64_t y, uint64_t bias, int mode);
/* the synchronous Linear of the backend on host buffers: x uploaded, the
 * weight from the cache, y downloaded (TInferCudaBackend.Linear,
 * backend.cuda.pas:469-515) */
int ihip_linear(ihip_ctx* ctx, const float* x, int64_t rows, int64_t in,
                const void* w, int dtype, int64_t out, const float* bias,
                float* y, int mode);

/* dequantize rows [row0, row0 + rows) of a repacked weight to F32
 * (InferRowToF32, tensor.pas:467-602, on the device) */
int ihip_enqueue_dequant(ihip_ctx* ctx, uint64_t w, int dtype, int64_t out,
                         int64_t in, int64_t row0, int64_t rows, uint64_t y);

/* ---- the operations of a layer (tools/cuda/ops.cu counterparts) ---- */

/* activations of `rows` rows quantized for IHIP_MODE_Q8 into the device
 * buffer xq (ihip_q8_bytes each): Q8_0 (k_quant 0) or Q8_K (k_quant 1) -
 * InferQuantizeRowQ8_0 / InferQuantizeRowQ8_K (backend.cpu.pas:617-819).
 * A non-finite value sets the int32 at `bad` (device address, may be 0) */
uint64_t ihip_q8_bytes(int64_t in, int k_quant);
int ihip_enqueue_quantize(ihip_ctx* ctx, uint64_t x, int64_t rows, int64_t in,
                          int k_quant, uint64_t xq, uint64_t bad);
/* y = w * x / sqrt(mean x^2 + eps) per row (TInferCpuBackend.RmsNorm,
 * backend.cpu.pas:1769-1795); y may be x */
int ihip_enqueue_rmsnorm(ihip_ctx* ctx, uint64_t x, uint64_t w, uint64_t y,
                         int64_t rows, int64_t cols, double eps);
/* x += t, then y = rmsnorm(x) (addnorm, ops.cu:135-150) */
int ihip_enqueue_addnorm(ihip_ctx* ctx, uint64_t x, uint64_t t, uint64_t w,
                         uint64_t y, int64_t rows, int64_t cols, double eps);
/* x += t */
int ihip_enqueue_add(ihip_ctx* ctx, uint64_t x, uint64_t t, int64_t n);
/* gate = silu(gate) * up, or the clamped gpt-oss form when limit > 0
 * (TInferCpuBackend.SwiGlu, backend.cpu.pas:1797-1834) */
int ihip_enqueue_swiglu(ihip_ctx* ctx, uint64_t gate, uint64_t up, int64_t n,
                        float alpha, float limit);
/* per row and head: RMSNorm of q/k heads (qn, kn device [head_dim] or 0),
 * rotate_half RoPE from cs = [rows, hd/2] cos then [rows, hd/2] sin, q in
 * place, k and v stored into the caches at row past + r
 * (qkrope, ops.cu:211-314; CPU: decoder.pas:2625-2680); kv_f16 selects a
 * half-float cache */
int ihip_enqueue_qkrope(ihip_ctx* ctx, uint64_t q, uint64_t k, uint64_t v,
                        uint64_t qn, uint64_t kn, uint64_t cs, uint64_t kc,
                        uint64_t vc, int64_t rows, int64_t heads,
                        int64_t kv_heads, int64_t head_dim, int64_t past,
                        double eps, int kv_f16);
/* causal GQA attention of `rows` new rows over the cache (window > 0: the
 * last `window` keys; sinks: device [heads] or 0; scale 0: 1/sqrt(hd))
 * (TInferCpuBackend.CausalAttention, backend.cpu.pas:1233-1380;
 * attention + attnmerge, ops.cu:352-617) */
int ihip_enqueue_attention(ihip_ctx* ctx, uint64_t q, uint64_t kc, uint64_t vc,
                           uint64_t y, int64_t rows, int64_t heads,
                           int64_t kv_heads, int64_t head_dim, int64_t past,
                           int64_t window, uint64_t sinks, double scale,
                           int kv_f16);
/* the router of TDecoderModel.Route (decoder.pas:2901-2949) for one row of
 * logits, on the device: ids and weights sorted by id (route, ops.cu:664-720);
 * scale (or 0): [experts] F32, each weight times its expert's after the
 * renorm (Gemma 4's per_expert_scale) */
int ihip_enqueue_route(ihip_ctx* ctx, uint64_t logits, int64_t experts,
                       int64_t k, int norm_topk, uint64_t ids, uint64_t w, uint64_t scale);
/* y = sum over slots in id order of w[s] * d[s] (moecombine, ops.cu:724-734) */
int ihip_enqueue_moecombine(ihip_ctx* ctx, uint64_t d, uint64_t w, uint64_t y,
                            int64_t k, int64_t n);
/* x[r] = InferRowToF32(embed, ids[r]) for device ids (TDecoderModel.Embed,
 * decoder.pas:2563-2580); embed is a repacked weight [vocab, hidden] */
int ihip_enqueue_embed(ihip_ctx* ctx, uint64_t embed, int dtype, int64_t vocab,
                       int64_t hidden, uint64_t ids, int64_t rows, uint64_t x);
/* the first index of the maximum of n floats, NaN skipped, lowest id on a tie
 * (InferArgMax, sampler.pas:123-160), written as int32 to `out` */
int ihip_enqueue_argmax(ihip_ctx* ctx, uint64_t v, int64_t n, uint64_t out);
/* a read-only streaming kernel over `bytes` at p (16-byte loads, every CU):
 * the achievable HBM read bandwidth, measured beside the GEMV (diagnostic,
 * no counterpart in the reference) */
int ihip_enqueue_stream_read(ihip_ctx* ctx, uint64_t p, uint64_t bytes, uint64_t out);

/* ======================================================================
 * TInferSampler (src/infer/mormot.ai.infer.sampler.pas:52-435) on the device
 * ==================================================================== */
typedef struct ihip_sampler ihip_sampler;

/* TInferSampling (sampler.pas:46-59): temperature <= 0 is greedy; top_k 0,
 * top_p 1 and min_p 0 filter nothing; the seed starts the splitmix64 stream */
typedef struct {
  double temperature;
  int32_t top_k;
  int32_t reserved;
  double top_p, min_p;
  int64_t seed;
} ihip_sampling;

/* the settings checked as TInferSampler.Create (sampler.pas:210-223), the
 * generator state and buffers for rows of up to n_max (at most 2^22) logits
 * on the device */
int ihip_sampler_create(ihip_ctx* ctx, const ihip_sampling* s, int64_t n_max, ihip_sampler** out);
void ihip_sampler_destroy(ihip_sampler* s);
/* the next token of n logits at `logits`, written as int32 to `out`
 * (TInferSampler.Next, sampler.pas:269-435): the argmax when greedy, else one
 * draw that advances the sampler's stream on the device (graph-capturable) */
int ihip_enqueue_sample(ihip_ctx* ctx, ihip_sampler* s, uint64_t logits, int64_t n, uint64_t out);

/* ======================================================================
 * TQwen3Cuda (src/infer/mormot.ai.infer.model.qwen3.cuda.pas:150-301):
 * the whole decoder on the device, behind TDecoderDevice
 * (src/infer/mormot.ai.infer.decoder.pas:907-928)
 * ==================================================================== */

/* one host tensor: data in the GGUF/safetensors layout of dtype, or NULL */
typedef struct {
  const void* data;
  int32_t dtype;
  int32_t reserved;
} ihip_tensor;

/* the weights of one layer (TDecoderLayer, decoder.pas:253-267) */
typedef struct {
  ihip_tensor input_norm;  /* [hidden] F32 */
  ihip_tensor q, k, v, o;  /* [qw, h], [kvw, h], [kvw, h], [h, qw] */
  ihip_tensor q_bias, k_bias, v_bias, o_bias; /* F32 or NULL (gpt-oss) */
  ihip_tensor q_norm, k_norm; /* [head_dim] F32 or NULL (Qwen3) */
  ihip_tensor sinks;       /* [heads] F32 or NULL (gpt-oss) */
  ihip_tensor post_norm;   /* [hidden] F32: the pre-FFN norm */
  ihip_tensor gate, up, down; /* dense FFN [ff, h], [ff, h], [h, ff] */
  ihip_tensor router, router_bias; /* [experts, h] and [experts] */
  ihip_tensor exp_gate, exp_up, exp_down; /* [E, fi, h], [E, fi, h], [E, h, fi] */
  ihip_tensor exp_gate_bias, exp_up_bias, exp_down_bias; /* [E, fi], [E, fi], [E, h] */
  int32_t window;          /* sliding window, 0 = full attention */
  int32_t moe;             /* 1: the FFN is a mixture of experts */
  /* Qwen3.5 (model.qwen35.pas:426-543, decoder.pas:2625-2855) */
  int32_t mixer;           /* IHIP_MIXER_ATTENTION or IHIP_MIXER_DELTANET */
  int32_t output_gate;     /* 1: q is [2 * heads * head_dim, h]: per head its
                              query rows, then its gate rows (Spec.OutputGate) */
  /* the Gated DeltaNet (mixer IHIP_MIXER_DELTANET): cd = 2 * key heads *
   * key dim + value heads * value dim channels, vd = value heads * value dim */
  ihip_tensor lin_qkv;     /* [cd, h]: the q, k and v channels */
  ihip_tensor lin_z;       /* [vd, h]: the output gate */
  ihip_tensor lin_b, lin_a; /* [value heads, h]: beta and the decay input */
  ihip_tensor lin_out;     /* [h, vd] */
  ihip_tensor lin_conv;    /* [cd, conv] F32: the depthwise causal convolution */
  ihip_tensor lin_dt_bias; /* [value heads] F32 */
  ihip_tensor lin_neg_a;   /* [value heads] F32: -exp(A_log) */
  ihip_tensor lin_norm;    /* [value dim] F32: the gated RMSNorm's weight */
  /* Gemma 4 (model.gemma4.pas:509-860, decoder.pas:2625-3091, :3245-3369) */
  int32_t head_dim, kv_heads; /* this layer's heads (0: the model's) */
  int32_t k_is_v;          /* 1: no v: the values are the raw keys (KIsV) */
  int32_t rope_set;        /* 0: the first rotary set, 1: the second (Rope2) */
  int32_t exp_gate_up;     /* 1: exp_gate is [E, 2 fi, h], per expert its gate
                              rows then its up rows; exp_up unused */
  int32_t no_rope;         /* 1: no rotary positions on q and k in this layer
                              (NoPE, TDecoderLayerSpec.NoRope, decoder.pas:139;
                              SmolLM3's no_rope_layers, model.qwen3.pas:28-33) */
  ihip_tensor attn_out_norm; /* [h] F32: the attention output normed before
                                the residual (SandwichNorm), or NULL */
  ihip_tensor ffn_out_norm;  /* [h] F32: the feed-forward output normed
                                before the residual, or NULL */
  /* moe == IHIP_FFN_DENSE_MOE (dfDenseMoe): the dense block's output norm,
   * the experts' input and output norms, the router input's norm weight
   * (an RMSNorm of the residual times it) and the expert scales */
  ihip_tensor dense_out_norm, moe_in_norm, moe_out_norm, router_norm;
  ihip_tensor expert_scale;  /* [E] F32: each route weight times its expert's */
  ihip_tensor scalar;        /* [1] F32: the layer's output state times it, or NULL */
} ihip_layer_desc;

/* ihip_layer_desc.moe (TDecoderFfn, decoder.pas:107-115) */
#define IHIP_FFN_DENSE 0
#define IHIP_FFN_MOE 1
#define IHIP_FFN_DENSE_MOE 2

/* ihip_layer_desc.mixer (TDecoderMixer, decoder.pas:95-105) */
#define IHIP_MIXER_ATTENTION 0
#define IHIP_MIXER_DELTANET 1

/* the settings of TDecoderConfig (decoder.pas:158-225) that this path reads */
typedef struct {
  int32_t vocab, hidden, layers, heads, kv_heads, head_dim;
  int32_t ffn, experts, experts_used, expert_ffn;
  int32_t norm_topk, max_positions;
  float rms_eps;
  float swiglu_alpha, swiglu_limit;
  float reserved0;
  double rope_theta;
  /* YaRN (decoder.pas:1759-1829): factor 0 = none */
  double rope_factor, rope_beta_fast, rope_beta_slow;
  int32_t rope_original, rope_truncate;
  double rope_attention;
  ihip_tensor embed, final_norm, head; /* head.data NULL: tied to embed */
  const ihip_layer_desc* layer;        /* [layers] */
  /* the rotating values of every head, from its start (RopeDims,
   * decoder.pas:216; 0: the whole head) */
  int32_t rope_dims;
  /* the DeltaNet shapes (decoder.pas:217-224), 0 without such a layer */
  int32_t lin_key_heads, lin_value_heads, lin_key_dim, lin_value_dim, lin_conv;
  /* LinTiled: value head h reads key head h mod key heads (llama.cpp's
   * order), else key head h / (value heads / key heads) */
  int32_t lin_tiled;
  /* Gemma 4 */
  int32_t activation;      /* IHIP_ACT_SILU (SwiGLU) or IHIP_ACT_GELU_TANH (GeGLU) */
  int32_t value_norm;      /* 1: every V head RMS-normed without weight */
  float embed_scale;       /* > 0: the embeddings of ids times it (single) */
  float reserved2;
  double attention_scale;  /* > 0: the score factor, else 1 / sqrt(head dim) */
  double logit_softcap;    /* > 0: logits := tanh(logits / c) * c */
  /* the second rotary set (Rope2Theta, decoder.pas:1742-1752): its theta, and
   * the rotating pairs from the start of its heads (the others keep
   * frequency 0) */
  double rope2_theta;
  int32_t rope2_pairs, reserved3;
} ihip_model_desc;

/* ihip_model_desc.activation (TDecoderActivation) */
#define IHIP_ACT_SILU 0
#define IHIP_ACT_GELU_TANH 1

/* the model on the device: every weight uploaded (UploadWeights,
 * model.qwen3.cuda.pas:602-828); mode: the Linear arithmetic; kv_f16: a
 * half-float KV cache (TQwen3Cuda.KvF16); max_tokens: the capacity of the
 * model's own context's cache up front (it grows beyond, up to
 * max_positions); the host tensors must outlive it */
int ihip_model_create(ihip_ctx* ctx, const ihip_model_desc* desc, int mode,
                      int kv_f16, int64_t max_tokens, ihip_model** out);
void ihip_model_destroy(ihip_model* m);
/* forget the cached tokens (TDecoderContext.Truncate(0)) */
int ihip_model_reset(ihip_model* m);
/* count tokens after the cached ones; logits [vocab] of the last one, or of
 * every one when all_logits (TQwen3Cuda.Forward, model.qwen3.cuda.pas:1722) */
int ihip_model_forward(ihip_model* m, const int32_t* ids, int64_t count,
                       float* logits, int all_logits);
/* greedy decode (TDecoderModel.Greedy, decoder.pas:3390-3426): the prompt,
 * then max_new ids by argmax; with the argmax on the device */
int ihip_model_greedy(ihip_model* m, const int32_t* prompt, int64_t n,
                      int64_t max_new, int32_t* out_ids);
/* steps greedy decode steps continuing the cache: token `first` (the last
 * id, not yet in the cache) enters it, out_ids[i] is the argmax after step i;
 * each step is one replay of the decode graph (the Forward(id, 1) of
 * TDecoderModel.Greedy, decoder.pas:3410-3422) */
int ihip_model_decode(ihip_model* m, int32_t first, int64_t steps, int32_t* out_ids);
/* the cos/sin table the model uploads for positions [first, first + rows):
 * [rows, rope/2] cos then sin (TDecoderModel.Rotary, decoder.pas:2539-2561) */
int ihip_model_rotary(const ihip_model_desc* desc, int64_t first, int64_t rows,
                      float* cs);
/* prompt rows per chunk of a forward pass: 1..1024 (default 1024); the
 * reference's CHUNK_MAX (model.qwen3.cuda.pas:308) is a constant 256 */
int ihip_model_chunk(ihip_model* m, int64_t rows);
/* how ihip_model_greedy and ihip_model_decode choose each next token: the
 * argmax (s NULL or temperature <= 0), or draws of a TInferSampler with these
 * settings, made on the device inside the decode graph (TNativeLlmClient's
 * sampling, llm.native.pas; the logits never leave the device) */
int ihip_model_sampling(ihip_model* m, const ihip_sampling* s);
/* decode steps as one replayed HIP graph (on, the default) or as direct
 * launches (TQwen3Cuda.UseGraphs, model.qwen3.cuda.pas:253-262) */
int ihip_model_use_graphs(ihip_model* m, int on);
/* CheckRoute (TQwen3Cuda.CheckRoute, model.qwen3.cuda.pas:288-300), a
 * diagnosis: with on, after every route the device forms for one row (the
 * decode steps' experts) the step waits, reads the router logits and the
 * choice back and compares them with TDecoderModel.Route on the same logits
 * on the host; the decode runs without graphs meanwhile */
int ihip_model_check_route(ihip_model* m, int on);
/* CheckRoute's counts (RouteChecks, RouteMismatches, RouteMaxDiff): rows
 * compared, rows whose ids differ, the largest weight difference of the rows
 * with the same ids (1e30 for a NaN or an infinity) */
int ihip_model_route_stats(ihip_model* m, int64_t* checks, int64_t* mismatches, double* max_diff);
/* TDecoderRouteTape in replay mode (decoder.pas:2955-3035; the reference's
 * device tests hand the CPU's expert choice to the device this way,
 * tests/test.infer.cuda.pas:2162-2200): ids / weights [rows][experts_used],
 * the picks (by id) and weights of every routed row of another run, given in
 * turn to the rows this model routes from now on (prompt rows and decode
 * steps, without graphs) in place of its own choice, which is compared with
 * them; rows 0: off. A row past the tape is refused. */
int ihip_model_route_tape(ihip_model* m, const int32_t* ids, const float* weights, int64_t rows);
/* A test hook (no counterpart in the reference): after each later chunk,
 * the residual rows [rows, hidden] after layer `layer` (0-based; -1: every
 * layer, [layers, rows, hidden]) copied to `rows` (host memory the caller
 * keeps alive; NULL turns it off). One-row decode steps on the fused path
 * are not captured. */
int ihip_model_debug_layer(ihip_model* m, int layer, float* rows);

/* the tape's counts: rows replayed, rows where the device's own choice
 * differed, the largest router gap (k-th chosen minus the best left out, in
 * the device's logits) of those rows, rows not yet replayed */
int ihip_model_route_tape_stats(ihip_model* m, int64_t* routes, int64_t* differs, double* gap,
                                int64_t* pending);
/* timings of the last greedy call: prefill and decode milliseconds */
int ihip_model_timing(ihip_model* m, double* prefill_ms, double* decode_ms);

/* ---- contexts of a model (TDecoderDevice, decoder.pas:907-928) ----
 * A context is one sequence on the device: its KV cache (grown as tokens
 * come: doubled, at least a quarter beyond them, up to max_positions -
 * Prepare, model.qwen3.cuda.pas:856-940), the id of each cached position, the
 * activations of a chunk and its own decode graph; the weights are the
 * model's, shared by all of its contexts. The ihip_model_* calls above use
 * the model's own context (ihip_model_context). One context at a time per
 * device (the calls take the device's lock). */
typedef struct ihip_mctx ihip_mctx;
/* a new, empty context (NewDeviceContext, model.qwen3.cuda.pas:229-231) */
int ihip_model_new_context(ihip_model* m, ihip_mctx** out);
/* free a context made by ihip_model_new_context (the model's own goes with it) */
void ihip_context_destroy(ihip_mctx* s);
/* the model's own context */
ihip_mctx* ihip_model_context(ihip_model* m);
/* Forward (model.qwen3.cuda.pas:1722-1730): count ids after the cached
 * tokens; logits [vocab] of the last one, or [count, vocab] with all_logits,
 * or NULL */
int ihip_context_forward(ihip_mctx* s, const int32_t* ids, int64_t count, float* logits,
                         int all_logits);
/* ForwardEmbeds (model.qwen3.cuda.pas:237-245, :1732-1739): count rows of
 * [hidden] floats in place of token embeddings; normed (or NULL) receives the
 * last row after the final norm [hidden]; head: the head of the logits (0,
 * the one head of these models; another is refused) */
int ihip_context_forward_embeds(ihip_mctx* s, const float* embeds, int64_t count, float* logits,
                                int all_logits, float* normed, int head);
/* Reuse (model.qwen3.cuda.pas:1741-1752): keep the cached tokens that start
 * ids, at most count - 1 of them (a position fed an embedding row matches no
 * id), drop the rest; *kept = the tokens kept */
int ihip_context_reuse(ihip_mctx* s, const int32_t* ids, int64_t count, int64_t* kept);
/* TDecoderContext.Truncate (decoder.pas:996-1016): keep the first length
 * tokens (the device keeps every row, so any length is restorable, but for
 * a model with DeltaNet layers: 0, the cached length, or a restore point) */
int ihip_context_truncate(ihip_mctx* s, int64_t length);
/* cached tokens and the cache's capacity (either pointer may be NULL) */
int ihip_context_length(ihip_mctx* s, int64_t* length, int64_t* capacity);
/* TDecoderContext.CheckpointId / MaxCheckpoints (decoder.pas:466-620,
 * :1019-1081): a context of a model with DeltaNet layers keeps its states
 * before every `id` token of an aligned forward (each part starting at the
 * sequence start or at an `id` token), the last `max` of them (4 by default,
 * DECODER_CHECKPOINTS); Reuse then takes the last one before the end of the
 * common start, Truncate goes back to any of them. id -1: none. Another id
 * drops the restore points. */
int ihip_context_set_checkpoints(ihip_mctx* s, int32_t id, int64_t max);
/* the lengths of the restore points held, the oldest first (at most cap of
 * them written); count: how many there are */
int ihip_context_checkpoints(ihip_mctx* s, int64_t* lengths, int64_t cap, int64_t* count);
/* ihip_model_greedy and ihip_model_decode on a context */
int ihip_context_greedy(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                        int32_t* out_ids);
int ihip_context_decode(ihip_mctx* s, int32_t first, int64_t steps, int32_t* out_ids);

/* ---- TNativeLlmClient's device side (src/mormot.ai.llm.native.pas) ----
 * The tokenizer, chat template and output parser stay the caller's; the
 * parser's stop is given as token ids. */
/* NativeDecode (llm.native.pas:2135-2185) on a context: the prompt's cached
 * start kept (Reuse), the rest computed, then draws of a fresh TInferSampler
 * (`sampling`, NULL or temperature <= 0: greedy) among the first draw_ids
 * rows of the logits (<= 0: the vocabulary; the ids a tokenizer has), each
 * drawn token fed back until one of stop_ids is drawn or max_new tokens are
 * out. The context is limited to max_positions, or max_context when smaller
 * and > 0: a longer prompt is refused, max_new is cut to what fits. The last
 * drawn token is not fed (the context holds n + count - 1 tokens).
 * out_ids[max_new] receives the tokens, *out_count their number, *reused the
 * prompt tokens kept from the cache, *stopped whether a stop id ended it
 * (reused and stopped may be NULL). */
int ihip_native_decode(ihip_mctx* s, const int32_t* prompt, int64_t n, int64_t max_new,
                       const ihip_sampling* sampling, int64_t draw_ids, const int32_t* stop_ids,
                       int64_t nstop, int64_t max_context, int32_t* out_ids, int64_t* out_count,
                       int64_t* reused, int* stopped);
/* TNativePromptCache (llm.native.pas:2192-2350): up to `slots` idle contexts
 * of a model kept between requests, least recently used first */
typedef struct ihip_prompt_cache ihip_prompt_cache;
int ihip_prompt_cache_create(ihip_model* m, int64_t slots, ihip_prompt_cache** out);
/* frees the idle contexts (a context acquired and not released stays the
 * caller's) */
void ihip_prompt_cache_destroy(ihip_prompt_cache* pc);
/* SetSlots: the least recently used beyond the new count are freed */
int ihip_prompt_cache_set_slots(ihip_prompt_cache* pc, int64_t slots);
/* Clear: every idle context freed */
int ihip_prompt_cache_clear(ihip_prompt_cache* pc);
/* Acquire: the idle context sharing the longest start with the prompt (its
 * last token excluded, as Reuse computes it again); with none shared and the
 * cache full, the least recently used; else a new context. The context is
 * the caller's until released. */
int ihip_prompt_cache_acquire(ihip_prompt_cache* pc, const int32_t* prompt, int64_t n, ihip_mctx** out);
/* Release: counts the request (a hit when reused > 0) and keeps the context
 * as the most recently used (with no slot it is freed; a full cache frees
 * its least recently used) */
int ihip_prompt_cache_release(ihip_prompt_cache* pc, ihip_mctx* s, int64_t reused);
/* the requests, hits and reused tokens counted so far, and the idle contexts
 * (any pointer may be NULL) */
int ihip_prompt_cache_stats(ihip_prompt_cache* pc, int64_t* requests, int64_t* hits, int64_t* reused,
                            int64_t* idle);

/* ======================================================================
 * GGUF v3 files (TGgufFile, src/infer/mormot.ai.infer.loader.gguf.pas:94-170)
 * and the decoder description of a llama.cpp file
 * (NewDecoderModelFromGguf, decoder.pas:3491-3510)
 * ==================================================================== */
typedef struct ihip_gguf ihip_gguf;

/* the metadata value types (TGgufType, loader.gguf.pas:57-70) */
enum {
  IHIP_GGUF_UINT8 = 0, IHIP_GGUF_INT8, IHIP_GGUF_UINT16, IHIP_GGUF_INT16, IHIP_GGUF_UINT32,
  IHIP_GGUF_INT32, IHIP_GGUF_FLOAT32, IHIP_GGUF_BOOL, IHIP_GGUF_STRING, IHIP_GGUF_ARRAY,
  IHIP_GGUF_UINT64, IHIP_GGUF_INT64, IHIP_GGUF_FLOAT64
};

/* one key/value pair, a view into the file (TGgufValue, loader.gguf.pas:73-87):
 * data is the value or the first array element; a string starts with its
 * 8-byte length */
typedef struct {
  const char* key;
  int32_t vtype, etype;
  int64_t count;
  const void* data;
} ihip_gguf_value;

/* one tensor (TInferTensor): row-major shape (GGUF lists ne0 first), dtype as
 * TInferDType, data inside the mapped file */
typedef struct {
  const char* name;
  int32_t dtype, ndim;
  int64_t shape[4];
  int64_t count, bytes;
  const void* data;
} ihip_gguf_tensor;

/* map and validate a file (TGgufFile.Create, loader.gguf.pas:318-323): every
 * defect of TGgufFile.Parse (:405-585) returns IHIP_E_FORMAT with the reason
 * in ihip_last_error(), nothing is read past the end */
int ihip_gguf_open(const char* path, ihip_gguf** out);
/* validate a copy of an in-memory content (TGgufFile.CreateFromContent, :325-330) */
int ihip_gguf_open_mem(const void* data, int64_t size, ihip_gguf** out);
/* unmap (TGgufFile.Destroy): the desc of ihip_gguf_model_desc dies with it */
void ihip_gguf_close(ihip_gguf* g);
/* TGgufFile.Alignment, length(Values), length(Tensors) */
int64_t ihip_gguf_alignment(const ihip_gguf* g);
int64_t ihip_gguf_value_count(const ihip_gguf* g);
int64_t ihip_gguf_tensor_count(const ihip_gguf* g);
/* Values[i] in file order */
int ihip_gguf_value_at(const ihip_gguf* g, int64_t i, ihip_gguf_value* out);
/* the index of a key, -1 when absent (Find / Has, :595-609) */
int64_t ihip_gguf_find(const ihip_gguf* g, const char* key);
/* typed access, IHIP_E_FORMAT when missing or of another type (Str, Int,
 * Float, Bool, BoolDef, :622-710); a string is a view of len bytes */
int ihip_gguf_str(const ihip_gguf* g, const char* key, const char** s, int64_t* len);
int ihip_gguf_int(const ihip_gguf* g, const char* key, int64_t* v);
int ihip_gguf_float(const ihip_gguf* g, const char* key, double* v);
int ihip_gguf_bool(const ihip_gguf* g, const char* key, int* v);
int ihip_gguf_bool_def(const ihip_gguf* g, const char* key, int def, int* v);
/* an array of fixed-size elements of type elem, count elements expected
 * (-1 = any): a view into the file (Floats32, Ints32, Bytes, :727-760) */
int ihip_gguf_array(const ihip_gguf* g, const char* key, int32_t elem, int64_t count,
                    const void** data, int64_t* n);
/* strings [first, first + n) of a string array (Strings, :712-725) */
int ihip_gguf_strings(const ihip_gguf* g, const char* key, int64_t first, int64_t n,
                      const char** s, int64_t* len);
/* Tensors[i] in file order; the index of a tensor or -1 (FindTensor, :762) */
int ihip_gguf_tensor_at(const ihip_gguf* g, int64_t i, ihip_gguf_tensor* out);
int64_t ihip_gguf_find_tensor(const ihip_gguf* g, const char* name);
/* the tensor checked against a type and row-major dims (Weight, :778-797) */
int ihip_gguf_weight(const ihip_gguf* g, const char* name, int32_t dtype, int32_t ndim,
                     const int64_t* dims, const void** data);
/* the decoder of a qwen3, qwen3moe or gpt-oss file, its settings from the
 * metadata and its tensors checked by name, shape, type and scales as
 * TQwen3Model / TQwen3MoeModel / TGptOssModel.LoadGgufConfig + LoadWeights do
 * (model.qwen3.pas:419-620, :797-846; model.gptoss.pas:331-475, :700-760):
 * block matrices point into the mapped file, norms and biases are F32 (BF16
 * and F16 ones widened exactly into memory of g). Valid while g is open;
 * pass it to ihip_model_create. */
int ihip_gguf_model_desc(ihip_gguf* g, const ihip_model_desc** out);

/* ======================================================================
 * seeded synthetic weights, written on the host (the generators of
 * tests/test.infer.fast.pas:144-260 generalised to every block type)
 * ==================================================================== */

/* blocks of dtype for a [rows, cols] matrix at dst: codes uniform over their
 * bit range, scales uniform in [2^lo_exp2, 2^hi_exp2] (fp16, or E8M0 for
 * MXFP4); threads: 0 = all cores */
int ihip_synth_blocks(void* dst, int dtype, int64_t rows, int64_t cols,
                      uint64_t seed, int lo_exp2, int hi_exp2, int threads);
/* weights ~ N(0, sigma) in dtype: F32/BF16 rounded, Q8_0 by the GGUF
 * writer's ties-away quantizer, Q4_K/Q6_K/MXFP4 by codes whose scales give
 * that spread */
int ihip_synth_normal(void* dst, int dtype, int64_t rows, int64_t cols,
                      uint64_t seed, float sigma, int threads);

#ifdef __cplusplus
}
#endif

#endif /* MORMOT_AI_HIP_H */
