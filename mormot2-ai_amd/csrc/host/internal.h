// internal.h - host-side internals of libmormot_ai_hip (C++17, HIP runtime).
#pragma once

#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/mormot_ai_hip.h"
#include "../layout.h"

namespace ihip {

// rows from which a Q8 Linear runs on the MFMA GEMM instead of 8-row GEMVs:
// below 80 rows the GEMVs are faster (a 32-token prompt of Qwen3-0.6B
// prefills 1.6x faster on them, a 128-token one 7% slower)
constexpr int GEMM_MIN_ROWS = 80;
// F32/BF16/F16 weights on the f64 GEMM from 16 rows: gpt-oss-20b's BF16
// attention matrices take 19.3 ms for a 32-token prefill there against 25.0
// on the 8-row GEMVs, 20.1 against 36.4 for 64 tokens
constexpr int GEMM_MIN_ROWS_FLOAT = 16;
// the GEMM's smallest chunk (one 16-row tile)
constexpr int GEMM_TILE_ROWS = 16;

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define IHIP_CHECK(call)                                   \
  do {                                                     \
    hipError_t e_ = (call);                                \
    if (e_ != hipSuccess) return ::ihip::hip_fail(e_, #call); \
  } while (0)

struct WeightEntry {
  const void* host;
  int dtype;
  uint64_t bytes;
  uint64_t dev;
  int64_t stride_rows = 0;  // weight_rows: the rows from one matrix to the next
};

struct Kernel {
  hipFunction_t f = nullptr;
};

// the module of one embedded code object
struct Module {
  hipModule_t mod = nullptr;
  std::unordered_map<std::string, hipFunction_t> fn;
};

}  // namespace ihip

// TInferSampler (sampler.pas:52-435) on the device: the settings, the
// splitmix64 state and the buffers of sample_probs / _compact / _pick
struct ihip_sampler {
  ihip_ctx* c = nullptr;
  double temperature = 0, top_p = 1, min_p = 0;
  int32_t top_k = 0;
  int64_t n_max = 0;
  std::vector<void*> mem;
  uint64_t state = 0, p = 0, bsum = 0, bq = 0, bcnt = 0, bmass = 0, cid = 0, ckey = 0, cp = 0;
};

// one device + one non-blocking stream + the embedded modules + the weight
// cache (TInferCuda + TInferCudaBackend of the reference)
struct ihip_ctx {
  int device = 0;
  int cus = 256;
  bool use_gemm = true;        // Q8 chunks of >= GEMM_MIN_ROWS rows on the MFMA GEMM (IHIP_GEMM=0: off)
  int gemm_min_rows = ihip::GEMM_MIN_ROWS;  // the smallest chunk on the GEMM (IHIP_GEMM_MIN_ROWS)
  // the smallest chunk of F32/BF16/F16 weights on the f64 GEMM
  // (IHIP_GEMM_MIN_ROWS_FLOAT)
  int gemm_min_rows_float = ihip::GEMM_MIN_ROWS_FLOAT;
  int gemv_blocks_per_cu = 2;  // one-row GEMV launches: blocks per CU at least (IHIP_GEMV_BLOCKS_PER_CU)
  int gemv_hold = 1;  // one-row GEMV launches: at most this many rounds of resident blocks (IHIP_GEMV_HOLD)
  bool use_gemm8 = true;  // 2..79 quantized rows on the int8 matrix cores, gemm8 (IHIP_GEMM8=0: the VALU gemv_rows)
  // MXFP4 prefill GEMMs on the scaled f8f6f4 matrix cores (IHIP_GEMM_F8=1)
  // rather than the int8 ones
  bool gemm_f8 = false;
  bool gemm_split = true;  // float-weight GEMMs of few tiles split over the sum (IHIP_GEMM_SPLIT=0: off)
  bool attn_mfma = true;  // prompt attention ranges on the f64 matrix cores (IHIP_ATTN_MFMA=0: VALU tiles of 8 rows)
  hipStream_t stream = nullptr;
  std::vector<ihip::Module> modules;
  std::unordered_map<std::string, hipFunction_t> kernels;
  std::unordered_map<std::string, int> resident;  // blocks of a kernel one CU holds at once
  std::vector<ihip::WeightEntry> weights;
  int weight_epoch = 0;
  std::vector<uint64_t> allocations;
  // scratch of the synchronous Linear and of the quantized activations
  uint64_t scratch_x = 0, scratch_x_bytes = 0;
  uint64_t scratch_y = 0, scratch_y_bytes = 0;
  uint64_t scratch_q = 0, scratch_q_bytes = 0;
  uint64_t scratch_bad = 0;
  uint64_t scratch_split = 0, scratch_split_bytes = 0;  // split sums of the float-weight GEMM
  uint64_t scratch_argmax = 0;  // [ARGMAX_PARTS] block results of argmax_part
  uint64_t scratch_attn = 0, scratch_attn_bytes = 0;
  uint64_t scratch_planes = 0, scratch_planes_bytes = 0;  // e4m3 activation planes (gemm_mxfp4_f8)
  // the device address of static_scratch.hip's array on this device
  // (ihip_enqueue_linear_at_static), read once at ihip_create
  uint64_t static_scratch = 0;
  bool capturing = false;
  hipGraph_t graphs[16] = {};
  hipGraphExec_t execs[16] = {};
  const void* slot_owner[16] = {};  // the model whose decode graph a slot holds
  hipEvent_t events[64] = {};
  // the kernel timer (ihip_kernel_timer): launches whose name starts with
  // timer_prefix carry a start and a stop event of their own dispatch
  std::string timer_prefix;
  std::vector<hipEvent_t> timer_events;  // pairs: start, stop
  std::vector<std::string> timer_names;  // the kernel of each pair in use
  size_t timer_used = 0;                 // pairs in use since the last read
  // a timing build's stamp buffers (ihip_trace_buffer)
  std::string trace_prefix;
  std::vector<uint64_t> trace_ptrs, trace_globals;
  size_t trace_used = 0;
  std::mutex lock;
};

namespace ihip {

hipFunction_t kernel(ihip_ctx* c, const char* name);
// the blocks of `block` threads of kernel `name` that one CU runs at once
int resident_blocks(ihip_ctx* c, const char* name, int block, size_t shmem = 0);
int launch(ihip_ctx* c, const char* name, dim3 grid, dim3 block, void* args, size_t shmem = 0);
// count matrices of out rows each, matrix e starting stride_rows rows after
// matrix e - 1 in the host tensor (the gate rows, or the up rows, of experts
// stored [E, 2 * out, in]): uploaded contiguous like ihip_weight's, cached by
// host address and stride
int weight_rows(ihip_ctx* c, const void* host, int t, int64_t out, int64_t in, int64_t count,
                int64_t stride_rows, uint64_t* dev);
// grows a scratch buffer to at least bytes (never while capturing)
int scratch(ihip_ctx* c, uint64_t& buf, uint64_t& cap, uint64_t bytes);

// repack [count, out, in] GGUF blocks into the HIP layout (multi-threaded)
void repack(const void* src, void* dst, int dtype, int64_t out, int64_t in, int64_t count);
// and back (tests of the layout)
void unpack(const void* src, void* dst, int dtype, int64_t out, int64_t in, int64_t count);

// the Linear dispatch shared by the public entry points and the model
// block results of the two-stage argmax
constexpr int ARGMAX_PARTS = 1024;

struct LinearCall {
  uint64_t x = 0;      // float activations [rows, in]
  uint64_t xq = 0;     // quantized activations (Q8 mode), 0: quantized here
  int64_t rows = 1, in = 0, out = 0;
  int dtype = 0;
  uint64_t w = 0, bias = 0, y = 0;
  int mode = IHIP_MODE_F32;
  uint64_t ids = 0;    // expert ids: slots = rows
  int64_t stride = 0;
  int x_per_slot = 0;
  int nexp = 0;        // experts behind ids (a bad id gives a zero row), 0: unchecked
  uint64_t items = 0;  // grouped experts: int4 work items (expert, start, count)
  uint64_t perm = 0;   // and the slots sorted by expert; rows = slots
  int64_t nitems = 0;
  int item_rows = 8;   // the most slots per item (moe_plan's chunk): 8, or 64 for the GEMM
  // fused SwiGLU: y = swiglu(x W^T + bias, x W2^T + bias2) (one row per block)
  uint64_t w2 = 0, bias2 = 0;
  float alpha = 1.0f, limit = 0.0f;
  // one row: the activation row is rmsnorm(x) * nw (eps) before the GEMV
  // (TInferCpuBackend.RmsNorm fused into the staging), in <= 4096
  uint64_t nw = 0;
  double eps = 0;
  // y[o] = res[o] + value (y may be res): the caller's residual add
  uint64_t res = 0;
  // combine: rows = slots, ids [slots] (<= 8), x [slots, in]; y [out] =
  // res + the slot-order sum of cw[s] * the expert rows (TDecoderModel.Experts)
  uint64_t cw = 0;
  // nseg > 1: one row through up to 3 matrices of this type in one launch,
  // matrix s = (wseg[s], oseg[s] outputs, yseg[s], bseg[s]); w/out/y/bias unused
  int nseg = 0;
  uint64_t wseg[3] = {}, bseg[3] = {}, yseg[3] = {};
  int64_t oseg[3] = {};
  // a two-type launch (a kernel for the pair must exist): matrices nseg1..
  // are of dtype2
  int dtype2 = 0, nseg1 = 0;
  // self-routing (one token's expert slots, rows = rk, one row per block):
  // rl the router logits [rexp]; each block takes its slot's expert by rank,
  // one block writes the picks (by id) to ids and their weights to rw
  uint64_t rl = 0, rw = 0;
  int rexp = 0, rk = 0, rnorm = 0;
  // a normed one-row float GEMV (the router) also writes its normed row
  // quantized here (Q8_K when xq_k8, else Q8_0), for the next launch
  uint64_t xq_out = 0;
  int xq_k8 = 0;
  // [rexp] per-expert weight scales (Gemma 4), or 0
  uint64_t rscale = 0;
  // the caller cannot allocate (ihip_enqueue_linear_at_static): no path
  // that grows the context's scratch
  bool no_alloc = false;
  bool batch_rows() const { return items != 0; }
};
// whether one launch can take matrices of types a then b (gemv_<a>_<b>_*)
bool gemv_pair(ihip_ctx* c, int a, int b, int mode, int64_t in);
int enqueue_linear(ihip_ctx* c, const LinearCall& call);
// whether a weight type with `in` inputs has a Linear kernel
bool linear_ok(int dtype, int64_t in);
// bytes of one quantized activation row (Q8_0 or Q8_K) of `in` values
uint64_t q8_row_bytes(int64_t in);
// reads the device address of the static scratch array for the current device
int static_scratch_init(ihip_ctx* c);
// gives up a context's hold on the device array (ihip_destroy)
void static_scratch_release(const ihip_ctx* c);
// whether enqueue_linear runs a Q8 chunk of this weight type on the MFMA GEMM
// (and takes grouped items of up to 64 slots)
bool gemm_runs(const ihip_ctx* c, int dtype, int mode);
// which activation quantizer a weight type needs in Q8 mode: -1 none (float
// weights), 0 Q8_0, 1 Q8_K
int q8_kind(int dtype);
int enqueue_quantize(ihip_ctx* c, uint64_t x, int64_t rows, int64_t in, int kind, uint64_t xq);
// flash-decoding attention: ranges of at most 128 keys per block, then a merge;
// part holds heads * rows * splits * (hd + 2) doubles; pastp: the position
// of row 0 in device memory (graph replay), or 0: past
int attention_splits(int64_t maxkeys);
// x += the k expert rows cd weighted by cw in slot order, then y = rmsnorm(x)
int enqueue_addnorm_moe(ihip_ctx* c, uint64_t x, uint64_t cd, uint64_t cw, int64_t k, uint64_t w,
                        uint64_t y, int64_t rows, int64_t cols, double eps);
// the decode step's attention of one row: head norms and RoPE of q and the
// new key (stored into the cache with its value) and the ranges in one
// launch, then attention_merge; part [heads, splits, hd + 2] doubles; hd 64
// or 128
struct AttnOne {
  uint64_t q = 0, k = 0, v = 0, qn = 0, kn = 0, cs = 0, kc = 0, vc = 0, y = 0, sinks = 0;
  uint64_t pastp = 0, part = 0;
  uint64_t done = 0;  // [heads] zeroed counters: the merge in the kernel's last block per head
  double scale = 0, eps = 0;
  int64_t heads = 0, kvh = 0, hd = 0, past = 0, window = 0;
  int splits = 1, f16 = 0;
};
int enqueue_attention_one(ihip_ctx* c, const AttnOne& o);
int enqueue_attention(ihip_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t y, uint64_t part,
                      int64_t rows, int64_t heads, int64_t kvh, int64_t hd, int64_t past,
                      uint64_t pastp, int64_t window, uint64_t sinks, double scale, int f16,
                      int splits);

}  // namespace ihip
