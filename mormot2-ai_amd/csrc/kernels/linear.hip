// linear.hip - dequant-fused GEMV for gfx950 (decode: 1 row; small batch: up
// to 8 rows per launch row-chunk), plain and expert-indexed (MoE).
//
// What it computes: y[r, o] = bias[o] + sum_i W[o, i] x[r, i] for W in the
// HIP layout of layout.h - the contract of TInferBackend.Linear
// (src/infer/mormot.ai.infer.backend.pas:59-75) and of the reference's
// EnqueueLinearAt / EnqueueLinearIds (backend.cuda.pas:338-412).
//
// Two arithmetics (template MODE):
//  - F32 (0): x in float, W dequantized in float, the block scale applied to
//    the group's sum - the contract of tools/cuda/linear.cu:1-6 (a tolerance
//    against the double Linear over InferRowToF32 weights);
//  - Q8 (1): x quantized per row (Q8_0 or Q8_K, by quantize.hip), exact
//    integer group sums by v_dot4_i32_i8, scales applied and summed in double -
//    TInferCpuBackend.Linear (backend.cpu.pas:1409-1566, 823-967); float
//    weights summed in double.
//
// Mapping to CDNA4: one wave64 covers 64 / LPR output rows; the LPR lanes of
// a row take its 32-value groups g = lane + k * LPR (k < U), so the lanes of
// a wave read one contiguous run of the codes region with 16-byte loads. The
// activation of a lane's groups stays in registers for every row the wave
// visits (R = 1), the waves walk the rows grid-stride. Lane sums meet in a
// register butterfly (wave_sum) within the LPR lanes. Q8 mode with K-quants: the 8
// groups of a super-block sit in 8 neighbouring lanes, whose integer sums
// are added exactly before the one double product of the super-block.
#include "formats.h"
#include "route.h"

namespace ihip {

// threads per block of every kernel here (the host launches 256): blockDim.x
// itself costs a vector load of the dispatch's hidden arguments, and a wait
// for it, before the first weight load
constexpr int NT = 256;

struct LinArgs {
  const uint8_t* w;    // matrix base (plain) or expert 0 (ids)
  const float* x;      // [rows, in] float activations
  const uint8_t* xq;   // [rows] quantized rows: int8[in] then float[G]
  const float* bias;   // [out], [experts, out] with ids, or null
  float* y;            // [rows or slots, out]
  const int* ids;      // [slots] expert ids, or null
  int64_t stride;      // bytes between experts
  int32_t out, in, rows, lpr;
  int32_t x_per_slot;  // ids: x row = slot / x_per_slot, or 0 when 0
  int32_t nexp;        // ids: the number of experts (an id outside 0..nexp-1 gives a zero row), 0: unchecked
  // grouped experts (a prompt chunk): work item blockIdx.y = (expert, start,
  // count <= 8) over perm, the slots sorted by expert; slot s reads x row
  // s / x_per_slot and writes y row s
  const int4* items;
  const int* perm;
  // fused SwiGLU: w2 the up projection (same layout, stride and experts as
  // w), bias2 its bias; y = swiglu(x W^T + bias, x W2^T + bias2), GeGLU
  // when limit < 0
  const uint8_t* w2;
  const float* bias2;
  float alpha, limit;
  int* bad;  // set to 1 + row when an activation quantized here is not finite
  // one-row blocks: the staged row is rmsnorm(x row) * nw when nw is set
  const float* nw;
  double eps;
  // y[o] = res[o] + value, the caller's residual add (y may be res)
  const float* res;
  // combine: slot s < kslots reads x row s and expert ids[s]; y[o] = res[o] +
  // the sum over the slots, in order, of cw[s] * value_s
  const float* cw;
  int32_t kslots;
  // matrices of one launch (R = 1, nseg > 1): blockIdx.y = matrix s with
  // weights wseg[s], oseg[s] outputs into yseg[s], bias bseg[s]
  int32_t nseg;
  const uint8_t* wseg[3];
  const float* bseg[3];
  float* yseg[3];
  int32_t oseg[3];
  int32_t nseg1;  // a two-type launch: matrices 0..nseg1-1 of the first type, the rest of the second
  // self-routing (a token's one-row expert launch): rl the row's router
  // logits, rexp experts, rk picks, rnorm NormTopK; each block takes the
  // expert of its slot by rank (ids unused as input), and block (0, 0) writes
  // the picks sorted by id to ids and their weights to rw (route of
  // TDecoderModel.Route) for the down projection
  const float* rl;
  float* rw;
  int32_t rexp, rk, rnorm, rpad;
  // each written weight times its expert's scale (Gemma 4), or null
  const float* rscale;
  // a normed one-row float GEMV (gemv_flt) also writes its normed row
  // quantized (Q8_K when xq_k8, else Q8_0) to xq_out [in] codes then [in / 32]
  // floats: the next launch over the same normed row takes it as given
  uint8_t* xq_out;
  int32_t xq_k8, xq_pad;
  // matrices of one launch in one index space of blocks (bstart[1] > 0):
  // blocks [bstart[s], bstart[s + 1]) take matrix s, so the blocks of every
  // matrix are dispatched in the first round (by blockIdx.y, the blocks of
  // a short matrix came after every block of the long one)
  int32_t bstart[4];
};

// the matrix of a block of a several-matrix launch (blockIdx.y, or its place
// in the one index space)
__device__ __forceinline__ int seg_of(const LinArgs& a)
{
  if (a.bstart[1] <= 0) return (int)blockIdx.y;
  const int b = (int)blockIdx.x;
  return (b >= a.bstart[1] ? 1 : 0) + (a.nseg > 2 && b >= a.bstart[2] ? 1 : 0);
}

// F32 mode: the group's contribution to the row sum. x: the 32 activations,
// sx their sum. Every code is turned into its exact value (signed, offset
// removed) before it multiplies x, as InferRowToF32 dequantizes it: a bias
// taken out afterwards through sx would leave the rounding of two large sums,
// which a large scale (an E8M0 exponent up to 255: 2^127) turns into garbage
// for a block of zero codes.
template <int F>
__device__ __forceinline__ float group_f32(const Raw& r, const float (&x)[32], float sx, int g)
{
  // the offset of the unsigned codes: q - 8 (Q4_0), q - 16 (Q5_0), q - 32
  // (Q6_K); Q8_0 and MXFP4 codes are signed bytes; Q5_1 and Q4_K keep their
  // unsigned codes and an affine term in sx (w = d q + m, d q - m)
  constexpr float off = F == DT_Q4_0 ? 8.0f : (F == DT_Q5_0 ? 16.0f : (F == DT_Q6_K ? 32.0f : 0.0f));
  constexpr bool sgn = (F == DT_Q8_0 || F == DT_MXFP4);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int hi = 0; hi < 2; hi++) {
    float part[2] = {0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const uint32_t c = code_bytes<F>(r, d, hi);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t b = (c >> (8 * i)) & 255u;
        const float cf = sgn ? (float)(int)(int8_t)b : (float)b - off;
        part[i & 1] = __builtin_fmaf(cf, x[16 * hi + 4 * d + i], part[i & 1]);
      }
    }
    acc[2 * hi] = part[0];
    acc[2 * hi + 1] = part[1];
  }
  if constexpr (F == DT_Q6_K) {  // (d * sc) * (q - 32) per half of 16 values
    const float d = half_to_float(r.d);
    const float ta = d * (float)(int)(int8_t)(r.a & 255u);
    const float tb = d * (float)(int)(int8_t)(r.a >> 8);
    return ta * (acc[0] + acc[1]) + tb * (acc[2] + acc[3]);
  }
  const float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  if constexpr (F == DT_Q8_0 || F == DT_Q4_0 || F == DT_Q5_0) {
    return half_to_float(r.a) * s;
  } else if constexpr (F == DT_MXFP4) {
    return e8m0_half(r.a) * s;
  } else if constexpr (F == DT_Q5_1) {
    return half_to_float(r.a & 0xffffu) * s + half_to_float(r.a >> 16) * sx;
  } else {  // Q4_K
    int sc, m;
    scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, m);
    const float d1 = half_to_float(r.q1.x & 0xffffu) * (float)sc;
    const float m1 = half_to_float(r.q1.x >> 16) * (float)m;
    return d1 * s - m1 * sx;
  }
}

// Q8 mode, 32-value block types: the group's exact term in double.
// xw: the 8 dwords of Q8_0 codes, dx the fp16 scale of the activation block
// (as float), sxq the sum of the 32 activation codes
template <int F>
__device__ __forceinline__ double group_q8(const Raw& r, const int (&xw)[8], float dx, int sxq)
{
  int s = 0;
#pragma unroll
  for (int hi = 0; hi < 2; hi++)
#pragma unroll
    for (int d = 0; d < 4; d++) s = sdot4((int)code_bytes<F>(r, d, hi), xw[4 * hi + d], s);
  double dxd = dx;
  if constexpr (F == DT_Q8_0) {
    return (double)s * ((double)half_to_float(r.a) * dxd);
  } else if constexpr (F == DT_MXFP4) {
    return (double)s * (mxfp4_q8_scale(r.a) * dxd);
  } else if constexpr (F == DT_Q4_0) {
    return (double)(s - 8 * sxq) * ((double)half_to_float(r.a) * dxd);
  } else if constexpr (F == DT_Q5_0) {
    return (double)(s - 16 * sxq) * ((double)half_to_float(r.a) * dxd);
  } else {  // Q5_1: d * q part, then m * dx * sum(qx) (LinearQ8_0 with aMins)
    double t = (double)s * ((double)half_to_float(r.a & 0xffffu) * dxd);
    return t + (double)half_to_float(r.a >> 16) * (dxd * (double)sxq);
  }
}

// Q8 mode, K-quants: the group's integer parts of the super-block sums
// (InferQ4KSumsPascal / InferQ6KSumsPascal, kernels.pas:229-333)
template <int F>
__device__ __forceinline__ void group_q8k(const Raw& r, const int (&xw)[8], int sxl, int sxh,
                                          int g, int& isum, int& msum)
{
  int sl = 0, sh = 0;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    sl = sdot4((int)code_bytes<F>(r, d, 0), xw[d], sl);
    sh = sdot4((int)code_bytes<F>(r, d, 1), xw[4 + d], sh);
  }
  if constexpr (F == DT_Q4_K) {
    int sc, m;
    scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, m);
    // |sums| < 2^16 and scales < 64: 24-bit products (full-rate multiplies)
    isum = __mul24(sc, sl + sh);
    msum = __mul24(m, sxl + sxh);
  } else {
    int sa = (int)(int8_t)(r.a & 255u), sb = (int)(int8_t)(r.a >> 8);
    isum = __mul24(sa, sl - 32 * sxl) + __mul24(sb, sh - 32 * sxh);
    msum = 0;
  }
}

template <int F>
__device__ __forceinline__ double superblock_q8k(const Raw& r, int isum, int msum, float dx)
{
  double dxd = dx;
  if constexpr (F == DT_Q4_K) {
    double hd = half_to_float(r.q1.x & 0xffffu), hm = half_to_float(r.q1.x >> 16);
    return (hd * dxd) * (double)isum - (hm * dxd) * (double)msum;
  } else {
    return ((double)half_to_float(r.d) * dxd) * (double)isum;
  }
}

constexpr bool is_float_type(int F) { return F == DT_F32 || F == DT_BF16 || F == DT_F16; }
constexpr bool is_k_quant(int F) { return F == DT_Q4_K || F == DT_Q6_K; }

// activations of one group: float (F32 mode and float weights) or Q8 codes
struct XGroup {
  float f[32];
  float sx;
  int w[8];
  float dx;
  int sl, sh;
  // MXFP4 one-row path: the codes as f16 pairs (value j, value j + 16)
  uint32_t h[16];
};

// the activation codes of a group as f16 pairs (x_j, x_16+j), j = 4d + i:
// the operand order of the MXFP4 code bytes (value j low, j + 16 high nibble)
__device__ __forceinline__ void half_pairs(XGroup& x)
{
#pragma unroll
  for (int d = 0; d < 4; d++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float lo = (float)(int)(int8_t)(x.w[d] >> (8 * i));
      const float hi = (float)(int)(int8_t)(x.w[4 + d] >> (8 * i));
      x.h[4 * d + i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Q8 mode, MXFP4, codes converted by the matrix-core-era conversion: every
// code byte to two f16 (the doubled E2M1 values, scale 2), dotted with the f16
// activation pairs. Every value is an integer below 2^11 and every partial sum
// one below 2^24, so the float sum is the exact integer group sum.
__device__ __forceinline__ double group_mxfp4_h(const Raw& r, const XGroup& x)
{
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    const uint32_t q = comp(r.q0, d);
    const half2_t w0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 2.0f, 0);
    const half2_t w1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 2.0f, 1);
    const half2_t w2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 2.0f, 2);
    const half2_t w3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 2.0f, 3);
    s0 = __builtin_amdgcn_fdot2(w0, __builtin_bit_cast(half2_t, x.h[4 * d]), s0, false);
    s1 = __builtin_amdgcn_fdot2(w1, __builtin_bit_cast(half2_t, x.h[4 * d + 1]), s1, false);
    s0 = __builtin_amdgcn_fdot2(w2, __builtin_bit_cast(half2_t, x.h[4 * d + 2]), s0, false);
    s1 = __builtin_amdgcn_fdot2(w3, __builtin_bit_cast(half2_t, x.h[4 * d + 3]), s1, false);
  }
  const int s = (int)s0 + (int)s1;
  return (double)s * (mxfp4_q8_scale(r.a) * (double)x.dx);
}

template <int F, int MODE>
__device__ __forceinline__ void load_x(const LinArgs& a, int64_t xrow, int g, int G, XGroup& x)
{
  if (MODE == 0 || is_float_type(F)) {
    const float4* p = (const float4*)(a.x + xrow * a.in + (int64_t)g * 32);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 t = p[k];
      x.f[4 * k] = t.x;
      x.f[4 * k + 1] = t.y;
      x.f[4 * k + 2] = t.z;
      x.f[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int k = 0; k < 32; k++) s += x.f[k];
    x.sx = s;
  } else {
    const uint8_t* row = a.xq + xrow * ((int64_t)a.in + 4 * (int64_t)G);
    const uint4* p = (const uint4*)(row + (int64_t)g * 32);
    uint4 u0 = p[0], u1 = p[1];
    x.w[0] = (int)u0.x; x.w[1] = (int)u0.y; x.w[2] = (int)u0.z; x.w[3] = (int)u0.w;
    x.w[4] = (int)u1.x; x.w[5] = (int)u1.y; x.w[6] = (int)u1.z; x.w[7] = (int)u1.w;
    x.dx = ((const float*)(row + a.in))[g];
    int sl = 0, sh = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      sl = sdot4(x.w[k], 0x01010101, sl);
      sh = sdot4(x.w[4 + k], 0x01010101, sh);
    }
    x.sl = sl;
    x.sh = sh;
  }
}

// the contribution of group g of row o (raw already loaded) against x
template <int F, int MODE>
__device__ __forceinline__ void group_term(const uint8_t* w, const Raw& raw, int64_t o, int g,
                                           int64_t in, const XGroup& x, float& accf,
                                           double& accd, int& isum, int& msum)
{
  if constexpr (is_float_type(F)) {
    float v[32];
    load_fgroup<F>(w, o, g, in, v);
    if constexpr (MODE == 0) {
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int k = 0; k < 32; k += 2) {
        p0 = __builtin_fmaf(v[k], x.f[k], p0);
        p1 = __builtin_fmaf(v[k + 1], x.f[k + 1], p1);
      }
      accf += p0 + p1;
    } else {
      // the exact float products summed in double, four chains interleaved
      double p[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 32; k++) p[k & 3] = __builtin_fma((double)v[k], (double)x.f[k], p[k & 3]);
      accd += (p[0] + p[1]) + (p[2] + p[3]);
    }
  } else if constexpr (MODE == 0) {
    accf += group_f32<F>(raw, x.f, x.sx, g);
  } else if constexpr (is_k_quant(F)) {
    group_q8k<F>(raw, x.w, x.sl, x.sh, g, isum, msum);
  } else {
    accd += group_q8<F>(raw, x.w, x.dx, x.sl + x.sh);
  }
}

// one row's total from its lanes; K-quant Q8: the exact super-block sums of 8
// lanes first. Returns the value in lane 0 of the row segment.
template <int F, int MODE>
__device__ __forceinline__ double row_total(int lpr, const Raw& hdr, float dxsb, bool has_sb,
                                            float accf, double accd, int isum, int msum, int g0)
{
  if constexpr (MODE == 0 && !is_float_type(F)) {
    return (double)wave_sum(accf, lpr);
  } else if constexpr (MODE == 0) {
    return (double)wave_sum(accf, lpr);
  } else if constexpr (is_k_quant(F)) {
    (void)g0;
    isum = wave_sum(isum, 8);
    msum = wave_sum(msum, 8);
    double t = has_sb ? superblock_q8k<F>(hdr, isum, msum, dxsb) : 0.0;
    return wave_sum(t, lpr);
  } else {
    return wave_sum(accd, lpr);
  }
}

// the value of row o against the lane's activation groups: the lanes of the
// row meet in row_total (lane 0 of the row segment holds it)
template <int F, int MODE, int U, bool HX = false>
__device__ __forceinline__ double row_value(const uint8_t* w, const Raw (&rawin)[U], int64_t o,
                                            bool valid, const XGroup (&xg)[U], int lr, int lpr,
                                            int G, int64_t in)
{
  Raw raw[U];
#pragma unroll
  for (int k = 0; k < U; k++) {
    raw[k] = rawin[k];
    if constexpr (F == DT_Q4_K) expand_header(raw[k]);  // the rows' loads are QH loads
  }
  if constexpr (HX) {
    static_assert(F == DT_MXFP4 && MODE == 1, "f16 pairs: MXFP4 in the Q8 arithmetic");
    double accd = 0.0;
#pragma unroll
    for (int k = 0; k < U; k++)
    {
      // every group is formed (a group past the row reads clamped codes and
      // a zeroed activation), its term kept or dropped by a select
      const double t = group_mxfp4_h(raw[k], xg[k]);
      accd += (valid && lr + k * lpr < G) ? t : 0.0;
    }
    return wave_sum(accd, lpr);
  } else if constexpr (MODE == 1 && is_k_quant(F)) {
    // lpr is a multiple of 8 and G of 8: the k-th groups of 8 aligned lanes
    // form one super-block. Its exact integer sums meet in all 8 lanes, each
    // lane forms the super-block's double term, adds its super-blocks in
    // order, and the super-block sets of a row (lpr / 8 of them) meet last.
    int is[U], ms[U];
#pragma unroll
    for (int k = 0; k < U; k++) {
      const int g = lr + k * lpr;
      float af = 0.f;
      double ad = 0.0;
      is[k] = ms[k] = 0;
      group_term<F, MODE>(w, raw[k], o, g, in, xg[k], af, ad, is[k], ms[k]);
      const bool ok = valid && g < G;
      is[k] = ok ? is[k] : 0;
      ms[k] = ok ? ms[k] : 0;
    }
#pragma unroll
    for (int k = 0; k < U; k++) {
      is[k] = wave_sum(is[k], 8);
      ms[k] = wave_sum(ms[k], 8);
    }
    double tot = 0.0;
#pragma unroll
    for (int k = 0; k < U; k++)
    {
      const double t = superblock_q8k<F>(raw[k], is[k], ms[k], xg[k].dx);
      tot += (valid && lr + k * lpr < G) ? t : 0.0;
    }
    if (lpr > 8) tot = tot + xpart<8>(tot);
    if (lpr > 16) tot = tot + xpart<16>(tot);
    if (lpr > 32) tot = tot + xpart<32>(tot);
    return tot;
  } else if constexpr (!is_float_type(F)) {
    // every group is formed (a group past the row reads clamped codes and a
    // zeroed activation) and its term kept or dropped by a select, with no
    // branch a group: adding +0.0 leaves a sum that starts at +0.0 as it is
    float accf = 0.f;
    double accd = 0.0;
#pragma unroll
    for (int k = 0; k < U; k++) {
      const int g = lr + k * lpr;
      const bool ok = valid && g < G;
      float af = 0.f;
      double ad = 0.0;
      int isum = 0, msum = 0;
      group_term<F, MODE>(w, raw[k], o, g, in, xg[k], af, ad, isum, msum);
      accf += ok ? af : 0.f;
      accd += ok ? ad : 0.0;
    }
    return row_total<F, MODE>(lpr, raw[0], 0.f, false, accf, accd, 0, 0, 0);
  } else {
    float accf = 0.f;
    double accd = 0.0;
#pragma unroll
    for (int k = 0; k < U; k++) {
      int g = lr + k * lpr;
      int isum = 0, msum = 0;
      if (valid && g < G) group_term<F, MODE>(w, raw[k], o, g, in, xg[k], accf, accd, isum, msum);
    }
    return row_total<F, MODE>(lpr, raw[0], 0.f, false, accf, accd, 0, 0, 0);
  }
}

// ------------------------------------------------- activation row in LDS
// An R = 1 block (256 threads, as the host launches it) stages its
// activations in LDS once; every wave then reads its lanes' groups from
// there. Q8 mode with quantized weights: the codes [n] then float dx[n / 32]
// (the quantized-row layout of quantize_q8_0 / quantize_q8_k), else the
// floats. A staging call takes n <= 8192 contiguous values: one row, or the
// rows of several slots back to back (no group crosses a row); with the
// fused rmsnorm (NORM) one row of n <= XN / 2.
constexpr int XB = 256;
constexpr int XN = 8192;  // values per staging call

template <int F, int MODE>
constexpr bool stage_q8() { return MODE == 1 && !is_float_type(F); }

template <int F, int MODE>
constexpr int xs_bytes() { return stage_q8<F, MODE>() ? XN + XN / 8 : 4 * XN; }

// a thread's share between the two staging phases: values (and norm weights)
struct XStage {
  float4 f[8];    // floats: 4 per slot; quantized here: 2 slots per 8-value quarter
  float4 g[8];    // the norm weights of the same values
  uint32_t d[9];  // a given quantized row, one dword per slot
};

// phase 1: the global loads. src: n floats (nw: their norm weights, or null);
// qsrc: a quantized row of n values instead (Q8 mode, no norm)
template <int F, int MODE, bool NORM>
__device__ __forceinline__ void stage_load(const float* src, const uint8_t* qsrc, int n,
                                           const float* nw, XStage& s)
{
  const int tid = threadIdx.x;
  const float4* p = (const float4*)src;
  const float4* pw = (const float4*)nw;
  if constexpr (!stage_q8<F, MODE>()) {
#pragma unroll
    for (int k = 0; k < (NORM ? 4 : 8); k++) {
      if (k * XB < (n >> 2)) {
        const int i = min(tid + k * XB, (n >> 2) - 1);
        s.f[k] = p[i];
        if constexpr (NORM) s.g[k] = pw[i];
      }
    }
  } else if (qsrc) {
    const int nd = (n + 4 * (n >> 5)) >> 2;
#pragma unroll
    for (int k = 0; k < 9; k++) {
      if (k * XB < nd) s.d[k] = ((const uint32_t*)qsrc)[min(tid + k * XB, nd - 1)];
    }
  } else {
#pragma unroll
    for (int k = 0; k < (NORM ? 2 : 4); k++) {
      const int q = min(tid + k * XB, (n >> 3) - 1);  // the quarter of 8 values (group q / 4)
      if (k * XB < (n >> 3)) {
        s.f[2 * k] = p[2 * q];
        s.f[2 * k + 1] = p[2 * q + 1];
        if constexpr (NORM) {
          s.g[2 * k] = pw[2 * q];
          s.g[2 * k + 1] = pw[2 * q + 1];
        }
      }
    }
  }
}

// the rmsnorm of the staged values in place, TInferCpuBackend.RmsNorm
// (backend.cpu.pas:1769-1795): the sum of squares in double over the block,
// inv = 1 / sqrt(mean + eps), w * (float)(x * inv). Every thread calls it.
template <int NV>
__device__ __forceinline__ void stage_norm(float (&v)[NV], const float (&w)[NV], const bool (&has)[NV],
                                           int n, double eps)
{
  __shared__ double red[XB / 64];
  double ss = 0;
#pragma unroll
  for (int j = 0; j < NV; j++)
    if (has[j]) {
      double d = v[j];
      ss = ss + d * d;
    }
  ss = wave_sum(ss, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = 0;
#pragma unroll
  for (int i = 0; i < XB / 64; i++) ss += red[i];
  const double inv = 1.0 / sqrt(ss / (double)n + eps);
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = w[j] * (float)((double)v[j] * inv);
}

__device__ __forceinline__ void unpack8(const float4& a, const float4& b, float* v)
{
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// the Q8 quantization of quarter q (8 consecutive values) of a row:
// InferQuantizeRowQ8_0 with 4 lanes a group (K8 false: the group's largest
// magnitude / 127, dx the scale rounded to half) or InferQuantizeRowQ8_K with
// 32 lanes a super-block (K8: the super-block's first value of the largest
// magnitude m, codes rint(-127 / m * v) at most 127, dx its inverse). The
// lanes of a group / super-block are aligned neighbours of one wave, all
// calling it.
template <bool K8>
__device__ __forceinline__ void quant_quarter(const float (&v)[8], int q, uint32_t& c0, uint32_t& c1,
                                              float& dx, bool& nonfinite)
{
  nonfinite = false;
  float amax = 0.f, m = 0.f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    nonfinite |= (float_bits(v[j]) & 0x7f800000u) == 0x7f800000u;
    float f = fabsf(v[j]);
    if (f > amax) {
      amax = f;
      m = v[j];
      idx = 8 * q + j;
    }
  }
  c0 = c1 = 0;
  dx = 0.f;
  if constexpr (!K8) {
    amax = fmaxf(amax, xpart<1>(amax));
    amax = fmaxf(amax, xpart<2>(amax));
    float d = amax / 127.0f;
    if (!(d < 2.9387359e-39f)) {
      float id = 1.0f / d;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        uint32_t c = (uint32_t)(int)__builtin_rintf(v[j] * id) & 255u;
        if (j < 4) c0 |= c << (8 * j);
        else c1 |= c << (8 * (j - 4));
      }
    }
    dx = half_to_float(float_to_half(d));
  } else {
    first_max<1>(amax, m, idx);
    first_max<2>(amax, m, idx);
    first_max<4>(amax, m, idx);
    first_max<8>(amax, m, idx);
    first_max<16>(amax, m, idx);
    if (!(amax < 3.7320437e-37f)) {
      float iscale = -127.0f / m;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        int ci = (int)__builtin_rintf(iscale * v[j]);
        if (ci > 127) ci = 127;
        uint32_t c = (uint32_t)ci & 255u;
        if (j < 4) c0 |= c << (8 * j);
        else c1 |= c << (8 * (j - 4));
      }
      dx = 1.0f / iscale;
    }
  }
}

// phase 2: into LDS (codes / dx, or floats at xs), normed first with NORM
// (one row of n values), quantized on the way when no quantized row was given
// - the arithmetic of quantize_q8_0 / quantize_q8_k (InferQuantizeRowQ8_0,
// InferQuantizeRowQ8_K) with 4 threads per group of 32 values. bad: set to
// badrow when a value is not finite.
template <int F, int MODE, bool NORM>
__device__ __forceinline__ void stage_store(const XStage& s, bool quantized, int n, double eps,
                                            uint8_t* xs, float* dxs, int* bad, int badrow)
{
  const int tid = threadIdx.x;
  if constexpr (!stage_q8<F, MODE>()) {
    constexpr int KF = NORM ? 4 : 8;  // float4 slots per thread
    float v[4 * KF], w[4 * KF];
    bool has[4 * KF];
#pragma unroll
    for (int k = 0; k < KF; k++) {
      has[4 * k] = has[4 * k + 1] = has[4 * k + 2] = has[4 * k + 3] = tid + k * XB < (n >> 2);
      v[4 * k] = s.f[k].x; v[4 * k + 1] = s.f[k].y; v[4 * k + 2] = s.f[k].z; v[4 * k + 3] = s.f[k].w;
      if constexpr (NORM) {
        w[4 * k] = s.g[k].x; w[4 * k + 1] = s.g[k].y; w[4 * k + 2] = s.g[k].z; w[4 * k + 3] = s.g[k].w;
      }
    }
    if constexpr (NORM) stage_norm<4 * KF>(v, w, has, n, eps);
#pragma unroll
    for (int k = 0; k < KF; k++)
      if (has[4 * k]) ((float4*)xs)[tid + k * XB] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  } else if (quantized) {
    const int nd = (n + 4 * (n >> 5)) >> 2;
#pragma unroll
    for (int k = 0; k < 9; k++) {
      int i = tid + k * XB;
      if (i < nd) ((uint32_t*)xs)[i] = s.d[k];
    }
  } else {
    const int G = n >> 5;
    constexpr int KQ = NORM ? 2 : 4;  // 8-value quarters per thread
    float vv[8 * KQ], ww[8 * KQ];
    bool hh[8 * KQ];
#pragma unroll
    for (int k = 0; k < KQ; k++) {
      const bool has = tid + k * XB < 4 * G;
      unpack8(s.f[2 * k], s.f[2 * k + 1], &vv[8 * k]);
      if constexpr (NORM) unpack8(s.g[2 * k], s.g[2 * k + 1], &ww[8 * k]);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        hh[8 * k + j] = has;
        if (!has) vv[8 * k + j] = 0.f;
      }
    }
    if constexpr (NORM) stage_norm<8 * KQ>(vv, ww, hh, n, eps);
#pragma unroll
    for (int k = 0; k < KQ; k++) {
      if (k * XB >= 4 * G) break;  // the same for the whole block
      const int q = tid + k * XB;
      const bool has = q < 4 * G;  // whole groups (and super-blocks) on each side
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = has ? vv[8 * k + j] : 0.f;
      bool nonfinite;
      uint32_t c0, c1;
      float dx;
      quant_quarter<is_k_quant(F)>(v, q, c0, c1, dx, nonfinite);
      if (nonfinite && bad) bad[0] = badrow;
      if (has) {
        ((uint2*)xs)[q] = make_uint2(c0, c1);
        if ((q & 3) == 0) dxs[q >> 2] = dx;
      }
    }
  }
}

// the lane's group gi (counted over the staged values) from LDS: codes at
// xs + 32 gi and dxs[gi], or floats at xs + 128 gi
template <int F, int MODE>
__device__ __forceinline__ void lds_x(const uint8_t* xs, const float* dxs, int gi, XGroup& x)
{
  if constexpr (!stage_q8<F, MODE>()) {
    const float4* p = (const float4*)(xs + gi * 128);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 t = p[k];
      x.f[4 * k] = t.x;
      x.f[4 * k + 1] = t.y;
      x.f[4 * k + 2] = t.z;
      x.f[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int k = 0; k < 32; k++) s += x.f[k];
    x.sx = s;
  } else {
    const uint4* p = (const uint4*)(xs + gi * 32);
    uint4 u0 = p[0], u1 = p[1];
    x.w[0] = (int)u0.x; x.w[1] = (int)u0.y; x.w[2] = (int)u0.z; x.w[3] = (int)u0.w;
    x.w[4] = (int)u1.x; x.w[5] = (int)u1.y; x.w[6] = (int)u1.z; x.w[7] = (int)u1.w;
    x.dx = dxs[gi];
    int sl = 0, sh = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      sl = sdot4(x.w[k], 0x01010101, sl);
      sh = sdot4(x.w[4 + k], 0x01010101, sh);
    }
    x.sl = sl;
    x.sh = sh;
  }
}

// the weight registers of the T tiles tb, tb + nw, ... of a wave step
template <int F, int U, int T, bool GLU>
__device__ __forceinline__ void load_tiles(const uint8_t* w, const uint8_t* w2, const Regions& rg,
                                           int64_t tb, int64_t nw, int rpw,
                                           int rsub, int lr, int lpr, int G, int64_t in,
                                           int64_t out, Raw (&raw)[T][U], Raw (&raw2)[T][U])
{
  if constexpr (is_float_type(F)) return;
  // every load is issued (a row or group past the end reads the last one, its
  // value unused), so the wait for the activation row ahead of them is exact
#pragma unroll
  for (int i = 0; i < T; i++) {
    const int64_t o = min((tb + (int64_t)i * nw) * rpw + rsub, out - 1);
#pragma unroll
    for (int k = 0; k < U; k++) {
      const int g = min(lr + k * lpr, G - 1);
      load_group<F, true, F == DT_Q4_K>(w, rg, o, G, g, in, raw[i][k]);
      if constexpr (GLU) load_group<F, true, F == DT_Q4_K>(w2, rg, o, G, g, in, raw2[i][k]);
    }
  }
}

// ------------------------------------------------------------------ kernel
// R = 1: one activation row, kept in registers. R = 8: up to 8 rows per
// blockIdx.y chunk, activations read per group (from L1/L2).
template <int F, int MODE, int U, int R, bool GLU, bool NORM>
__device__ __forceinline__ void gemv(const LinArgs& a)
{
  IHIP_STAMP_SCOPE;
  const int lane = threadIdx.x & 63;
  const int lpr = a.lpr;
  const int lr = lane & (lpr - 1);
  const int rsub = lane / lpr;
  const int rpw = 64 / lpr;
  const int G = a.in >> 5;
  const uint8_t* w = a.w;
  const float* bias = a.bias;
  int out = a.out;
  float* yp = a.y;
  int bx = (int)blockIdx.x, gx = (int)gridDim.x;  // the block among its matrix's
  int64_t xrow0, yrow0;
  int nrows;
  int pstart = -1;  // grouped: the first entry of perm
  int64_t expert = 0;
  if (a.items) {
    const int4 it = a.items[blockIdx.y];
    if (it.z <= 0) return;
    expert = it.x;
    w += (int64_t)it.x * a.stride;
    if (bias) bias += (int64_t)it.x * a.out;
    pstart = it.y;
    nrows = min(R, it.z);
    xrow0 = yrow0 = 0;
  } else if (a.ids) {
    const bool routed = R == 1 && GLU && a.rl != nullptr;
    // a self-routed token: row 0 of the launch forms the route, row 1 + s
    // computes slot s
    const int slot = routed ? (int)blockIdx.y - 1 : (int)blockIdx.y;
    if (routed && slot < 0) {
      // the route row (dispatched first): wave 0 of its first block writes
      // the picks (by id) and their weights for the down launch, beside the
      // blocks of the slots
      if (blockIdx.x == 0 && threadIdx.x < 64) {
        int sid[8];
        float sw[8], lg[4];
        route_logits(a.rl, a.rexp, lg);
        if (a.rexp <= 64) route_wave<1, true>(lg, a.rexp, a.rk, a.rnorm, sid, sw);
        else if (a.rexp <= 128) route_wave<2, true>(lg, a.rexp, a.rk, a.rnorm, sid, sw);
        else route_wave<4, true>(lg, a.rexp, a.rk, a.rnorm, sid, sw);
        int myid = -1;
        float myw = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < 8; s2++) {
          myid = (int)threadIdx.x == s2 ? sid[s2] : myid;
          myw = (int)threadIdx.x == s2 ? sw[s2] : myw;
        }
        if ((int)threadIdx.x < a.rk) {
          if (a.rscale) myw = myw * a.rscale[myid];
          ((int*)a.ids)[threadIdx.x] = myid;
          a.rw[threadIdx.x] = myw;
        }
      }
      return;
    }
    // a self-routed token (one row) takes its expert below, once the
    // activation row is on its way
    const bool later = routed;
    const int e = later ? 0 : a.ids[slot];
    if (!later && (e < 0 || (a.nexp > 0 && e >= a.nexp))) {
      for (int64_t o = (int64_t)(blockIdx.x * NT + threadIdx.x); o < a.out;
           o += (int64_t)gridDim.x * NT)
        a.y[(int64_t)slot * a.out + o] = 0.f;
      return;
    }
    expert = e;
    w += (int64_t)e * a.stride;
    if (bias) bias += (int64_t)e * a.out;
    xrow0 = a.x_per_slot ? slot / a.x_per_slot : 0;
    yrow0 = slot;
    nrows = 1;
  } else if (R == 1 && a.nseg > 1) {
    // several matrices of this type over the same row
    const int sg = seg_of(a);
    if (a.bstart[1] > 0) {
      bx -= a.bstart[sg];
      gx = a.bstart[sg + 1] - a.bstart[sg];
    }
    w = a.wseg[sg];
    bias = a.bseg[sg];
    out = a.oseg[sg];
    yp = a.yseg[sg];
    xrow0 = yrow0 = 0;
    nrows = 1;
  } else {
    xrow0 = (int64_t)blockIdx.y * R;
    yrow0 = xrow0;
    nrows = min(R, a.rows - (int)xrow0);
  }
  const Regions rg = regions(F, out, a.in);
  const int64_t tiles = ((int64_t)out + rpw - 1) / rpw;
  const int64_t nw = (int64_t)gx * (NT >> 6);
  const int64_t wid = (int64_t)bx * (NT >> 6) + (threadIdx.x >> 6);

  if constexpr (R == 1) {
    IHIP_STAMP(0);
    if ((int64_t)bx * (NT >> 6) >= tiles) return;  // the whole block: no tile
    // T tiles per wave step, their weight loads issued together (and the
    // first ones before the activation row is read), so a wave keeps several
    // 16-byte loads per lane in flight
    constexpr int T = GLU ? (U == 1 ? 2 : 1) : (U == 1 ? 4 : (U == 2 ? 2 : 1));
    // the activation row's global loads first, then the first step's weight
    // loads, so the row is staged while the weights are on their way
    // a self-routed token: the router logits first (the route needs them
    // before any weight address is known)
    // (more than 64 experts: wave 0 alone, the other waves take its pick
    // from LDS - every wave of every block loading the same logit lines
    // queued them at the L2; with fewer, the barrier costs more than the
    // shared lines)
    float rlg[4];
    const bool shared_pick = a.rexp > 64;
    const bool route0 = !shared_pick || threadIdx.x < 64;
    if (GLU && a.ids && a.rl && route0) route_logits(a.rl, a.rexp, rlg);
    XStage st;
    const bool quantized = !NORM && stage_q8<F, MODE>() && a.xq != nullptr;
    stage_load<F, MODE, NORM>(a.x + xrow0 * a.in,
                              quantized ? a.xq + xrow0 * (int64_t)(a.in + 4 * G) : nullptr, a.in,
                              a.nw, st);
    IHIP_STAMP(6);
    if (GLU && a.ids && a.rl) {
      // self-routed (TDecoderModel.Route in the wave, route_wave): the expert
      // of this block's slot; the launch's extra row writes the picks and
      // weights for the down launch
      __shared__ int spick;
      int e = -1;
      if (route0) {
        int sid[8];
        float sw[8];
        if (a.rexp <= 64) route_wave<1, false>(rlg, a.rexp, a.rk, a.rnorm, sid, sw);
        else if (a.rexp <= 128) route_wave<2, false>(rlg, a.rexp, a.rk, a.rnorm, sid, sw);
        else route_wave<4, false>(rlg, a.rexp, a.rk, a.rnorm, sid, sw);
        int e0 = -1;
#pragma unroll
        for (int s = 0; s < 8; s++) e0 = s == (int)yrow0 ? sid[s] : e0;
        if (threadIdx.x == 0) spick = e0;
        if (!shared_pick) e = e0;
      }
      if (shared_pick) {
        __syncthreads();
        e = spick;
      }
      IHIP_STAMP(7);
      if (e < 0 || (a.nexp > 0 && e >= a.nexp)) {
        for (int64_t o = (int64_t)(blockIdx.x * NT + threadIdx.x); o < a.out;
             o += (int64_t)gridDim.x * NT)
          a.y[yrow0 * a.out + o] = 0.f;
        return;
      }
      expert = e;
      w += (int64_t)e * a.stride;
      if (bias) bias += (int64_t)e * a.out;
    }
    // gate + up + SwiGLU in one pass: w2 the up matrices, the same expert
    const uint8_t* w2 = GLU ? a.w2 + (w - a.w) : nullptr;
    const float* bias2 = a.bias2 ? a.bias2 + expert * out : nullptr;
    XGroup xg[U];
    Raw raw[T][U], raw2[T][U];
    __shared__ __align__(16) uint8_t xs[xs_bytes<F, MODE>()];
    constexpr bool HXP = F == DT_MXFP4 && MODE == 1;  // f16 activation pairs
    int64_t tb = wid;
    // the epilogue operands of a step's rows (bias, up bias, residual), loaded
    // with its weights rather than after its sums; a launch without them
    // issues no load for them (a uniform branch)
    float eb[T], eb2[T], er[T];
    auto load_epi = [&](int64_t sb) {
#pragma unroll
      for (int i = 0; i < T; i++) {
        const int64_t o = min((sb + (int64_t)i * nw) * rpw + rsub, (int64_t)out - 1);
        eb[i] = eb2[i] = er[i] = 0.f;
        if (bias) eb[i] = bias[o];
        if constexpr (GLU)
          if (bias2) eb2[i] = bias2[o];
        if (a.res) er[i] = a.res[o];
      }
    };
    load_tiles<F, U, T, GLU>(w, w2, rg, tb, nw, rpw, rsub, lr, lpr, G, a.in, out, raw,
                             raw2);
    load_epi(tb);
    IHIP_STAMP(1);
    stage_store<F, MODE, NORM>(st, quantized, a.in, a.eps, xs, (float*)(xs + a.in), a.bad,
                         1 + (int)xrow0);
    __syncthreads();
    IHIP_STAMP(2);
#pragma unroll
    for (int k = 0; k < U; k++) {
      int g = lr + k * lpr;
      xg[k] = XGroup{};
      if (g < G) lds_x<F, MODE>(xs, (const float*)(xs + a.in), g, xg[k]);
      if constexpr (HXP) half_pairs(xg[k]);
    }
    // the T tiles of a step from their weight registers
    auto step = [&](int64_t sb, const Raw (&rw)[T][U], const Raw (&rw2)[T][U]) {
#pragma unroll
      for (int i = 0; i < T; i++) {
        const int64_t t = sb + (int64_t)i * nw;
        const int64_t o = t * rpw + rsub;
        const bool valid = t < tiles && o < out;
        double v = row_value<F, MODE, U, HXP>(w, rw[i], o, valid, xg, lr, lpr, G, a.in);
        double v2 = 0.0;
        if constexpr (GLU) v2 = row_value<F, MODE, U, HXP>(w2, rw2[i], o, valid, xg, lr, lpr, G, a.in);
        if (lr == 0 && valid) {
          if (bias) v = (double)eb[i] + v;
          float r = (float)v;
          if constexpr (GLU) {
            if (bias2) v2 = (double)eb2[i] + v2;
            r = glu_value(r, (float)v2, a.alpha, a.limit);
          }
          if (a.res) r = er[i] + r;
          yp[yrow0 * out + o] = r;
        }
      }
    };
    IHIP_STAMP(3);
    while (tb < tiles) {
      step(tb, raw, raw2);
      IHIP_STAMP(4);
      tb += (int64_t)T * nw;
      if (tb < tiles) {
        load_tiles<F, U, T, GLU>(w, w2, rg, tb, nw, rpw, rsub, lr, lpr, G, a.in, out, raw, raw2);
        load_epi(tb);
      }
    }
    IHIP_STAMP(5);
  } else {
    // the activation and output rows of the batch
    int64_t xr[R], yr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (pstart >= 0) {
        int s = a.perm[pstart + min(r, nrows - 1)];  // (a row past the item: its last slot, unused)
        xr[r] = a.x_per_slot ? s / a.x_per_slot : 0;
        yr[r] = s;
      } else {
        xr[r] = xrow0 + r;
        yr[r] = yrow0 + r;
      }
    }
    for (int64_t t = wid; t < tiles; t += nw) {
      int64_t o = t * rpw + rsub;
      bool valid = o < out;
      float accf[R];
      double accd[R], tot[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        accf[r] = 0.f;
        accd[r] = 0.0;
        tot[r] = 0.0;
      }
#pragma unroll
      for (int k = 0; k < U; k++) {
        int g = lr + k * lpr;
        bool has = valid && g < G;
        Raw raw;
        if (has && !is_float_type(F)) load_group<F>(w, rg, o, G, g, a.in, raw);  // re-read per row chunk
#pragma unroll
        for (int r = 0; r < R; r++) {
          if (r < nrows) {
            int isum = 0, msum = 0;
            XGroup xg;
            if (has) {
              load_x<F, MODE>(a, xr[r], g, G, xg);
              group_term<F, MODE>(w, raw, o, g, a.in, xg, accf[r], accd[r], isum, msum);
            }
            if constexpr (MODE == 1 && is_k_quant(F)) {
              bool lead = (g & 7) == 0 && has;
              tot[r] += row_total<F, MODE>(lpr, raw, has ? xg.dx : 0.f, lead, 0.f, 0.0, isum,
                                           msum, g);
            }
          }
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (r < nrows) {
          double v;
          if constexpr (MODE == 1 && is_k_quant(F))
            v = tot[r];
          else
            v = row_total<F, MODE>(lpr, Raw{}, 0.f, false, accf[r], accd[r], 0, 0, 0);
          if (lr == 0 && valid) {
            if (bias) v = (double)bias[o] + v;
            yp[yr[r] * out + o] = (float)v;
          }
        }
      }
    }
  }
}

// -------------------------------------------------- rows of a small batch
// Q8 mode, quantized weights, up to RB = 8 activation rows per block
// (blockIdx.y: a chunk of 8 rows, or a grouped-expert work item): the rows'
// quantized codes, their scales and the sums of each half group staged in
// LDS once per block; every weight group is loaded once and decoded once
// into registers, then dotted with each row's group from LDS. The
// arithmetic per row is the one-row GEMV's (exact integer group or
// super-block sums, the scales in double, the same reduction order), so a
// batch row gives the bits of that row alone.
constexpr int RB = 8;

// bytes of one staged row: codes [in], dx [G] floats, half sums [G] int2
__host__ __device__ constexpr int rows_stride(int in) { return ((in + 12 * (in / 32)) + 15) & ~15; }

// one row's activation group from the stage
struct XRow {
  int w[8];
  float dx;
  int sl, sh;
};

// SUMS: the half sums are read too (the types with an offset or a min)
template <bool SUMS>
__device__ __forceinline__ void stage_xrow(const uint8_t* row, int G, int g, XRow& x)
{
  const uint4* p = (const uint4*)(row + g * 32);
  const uint4 u0 = p[0], u1 = p[1];
  x.w[0] = (int)u0.x; x.w[1] = (int)u0.y; x.w[2] = (int)u0.z; x.w[3] = (int)u0.w;
  x.w[4] = (int)u1.x; x.w[5] = (int)u1.y; x.w[6] = (int)u1.z; x.w[7] = (int)u1.w;
  x.dx = ((const float*)(row + 32 * G))[g];
  if constexpr (SUMS) {
    const int2 hs = ((const int2*)(row + 36 * G))[g];
    x.sl = hs.x;
    x.sh = hs.y;
  } else {
    x.sl = x.sh = 0;
  }
}

// the 8 code dwords of a group, decoded once for every row
template <int F>
__device__ __forceinline__ void decode_codes(const Raw& r, uint32_t (&cw)[8])
{
#pragma unroll
  for (int hi = 0; hi < 2; hi++)
#pragma unroll
    for (int d = 0; d < 4; d++) cw[4 * hi + d] = code_bytes<F>(r, d, hi);
}

template <int F, int U, int TB>
__device__ __forceinline__ void gemv_rows(const LinArgs& a)
{
  extern __shared__ __align__(16) uint8_t xst[];
  const int lane = threadIdx.x & 63;
  const int lpr = a.lpr;
  const int lr = lane & (lpr - 1);
  const int rsub = lane / lpr;
  const int rpw = 64 / lpr;
  const int G = a.in >> 5;
  const int RS = rows_stride(a.in);
  constexpr bool SUMS = !(F == DT_Q8_0 || F == DT_MXFP4);
  const uint8_t* w = a.w;
  const float* bias = a.bias;
  int nrows;
  int64_t xr[RB], yr[RB];
  if (a.items) {
    const int4 it = a.items[blockIdx.y];
    if (it.z <= 0) return;
    w += (int64_t)it.x * a.stride;
    if (bias) bias += (int64_t)it.x * a.out;
    nrows = min(RB, it.z);
#pragma unroll
    for (int r = 0; r < RB; r++) {
      // every load issued before the first is used (a row past the item's
      // reads its last slot, unused)
      const int sl = a.perm[it.y + min(r, nrows - 1)];
      xr[r] = a.x_per_slot ? sl / a.x_per_slot : 0;
      yr[r] = sl;
    }
  } else {
    const int64_t r0 = (int64_t)blockIdx.y * RB;
    nrows = min(RB, a.rows - (int)r0);
#pragma unroll
    for (int r = 0; r < RB; r++) xr[r] = yr[r] = r0 + r;
  }
  const Regions rg = regions(F, a.out, a.in);
  const int64_t tiles = ((int64_t)a.out + rpw - 1) / rpw;
  const int64_t nw = (int64_t)gridDim.x * (NT >> 6);
  const int64_t wid = (int64_t)blockIdx.x * (NT >> 6) + (threadIdx.x >> 6);
  Raw cur[TB][U], nxt[TB][U];
  // the weights of a step: TB tiles, every load issued before the first use
  auto load = [&](int64_t sb, Raw (&raw)[TB][U]) {
#pragma unroll
    for (int i = 0; i < TB; i++) {
      const int64_t o = min((sb + (int64_t)i * nw) * rpw + rsub, (int64_t)a.out - 1);
#pragma unroll
      for (int k = 0; k < U; k++) {
        const int g = min(lr + k * lpr, G - 1);
        load_group<F, true, F == DT_Q4_K>(w, rg, o, G, g, a.in, raw[i][k]);
      }
    }
  };
  int64_t tb = wid;
  // the stage: each thread takes groups of the rows (16-byte loads of the
  // codes, the half sums formed here once)
  const int64_t qstride = (int64_t)a.in + 4 * (int64_t)G;
  for (int t = threadIdx.x; t < nrows * G; t += NT) {
    const int r = t / G, g = t - r * G;
    const uint8_t* src = a.xq + xr[r] * qstride;
    const uint4 u0 = *(const uint4*)(src + g * 32), u1 = *(const uint4*)(src + g * 32 + 16);
    const float dx = ((const float*)(src + a.in))[g];
    int sl = 0, sh = 0;
    sl = sdot4((int)u0.x, 0x01010101, sl); sl = sdot4((int)u0.y, 0x01010101, sl);
    sl = sdot4((int)u0.z, 0x01010101, sl); sl = sdot4((int)u0.w, 0x01010101, sl);
    sh = sdot4((int)u1.x, 0x01010101, sh); sh = sdot4((int)u1.y, 0x01010101, sh);
    sh = sdot4((int)u1.z, 0x01010101, sh); sh = sdot4((int)u1.w, 0x01010101, sh);
    uint8_t* dst = xst + r * RS;
    *(uint4*)(dst + g * 32) = u0;
    *(uint4*)(dst + g * 32 + 16) = u1;
    ((float*)(dst + 32 * G))[g] = dx;
    ((int2*)(dst + 36 * G))[g] = make_int2(sl, sh);
  }
  __syncthreads();
  if (wid >= tiles) return;  // after the stage: every thread took its share
  load(tb, cur);
  while (tb < tiles) {
    const int64_t nb = tb + (int64_t)TB * nw;
    // the next step's weights in flight while this one is computed
    if (nb < tiles) load(nb, nxt);
#pragma unroll
    for (int i = 0; i < TB; i++) {
      const int64_t t = tb + (int64_t)i * nw;
      const int64_t o = t * rpw + rsub;
      const bool valid = t < tiles && o < a.out;
      uint32_t cw[U][8];
      Raw raw[U];
#pragma unroll
      for (int k = 0; k < U; k++) {
        raw[k] = cur[i][k];
        if constexpr (F == DT_Q4_K) expand_header(raw[k]);
        decode_codes<F>(raw[k], cw[k]);
      }
      float bo = 0.f;
      if (bias && valid) bo = bias[o];
      // the per-group weight factors of the K-quants, once for all rows
      int ksc[U], km[U];
#pragma unroll
      for (int k = 0; k < U; k++) {
        if constexpr (F == DT_Q4_K) {
          scale_min_k4((lr + k * lpr) & 7, raw[k].q1.y, raw[k].q1.z, raw[k].q1.w, ksc[k], km[k]);
        } else {
          ksc[k] = (int)(int8_t)(raw[k].a & 255u);
          km[k] = (int)(int8_t)(raw[k].a >> 8);
        }
      }
      if (nrows > 1) {
        // every row's partial sums at once, reduced transposed: the lane
        // ends with one row (rows_sum8), lanes 0..7 of the segment store
        double vr[RB];
        int n, base;
        if constexpr (is_k_quant(F)) {
          double tot = 0.0;
#pragma unroll
          for (int k = 0; k < U; k++) {
            const int g = lr + k * lpr;
            const int gc = min(g, G - 1);
            int isr[RB], msr[RB];
#pragma unroll
            for (int r = 0; r < RB; r++) {
              isr[r] = msr[r] = 0;
              if (r < nrows) {
                XRow xg;
                stage_xrow<SUMS>(xst + r * RS, G, gc, xg);
                int sl = 0, sh = 0;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                  sl = sdot4((int)cw[k][d], xg.w[d], sl);
                  sh = sdot4((int)cw[k][4 + d], xg.w[4 + d], sh);
                }
                if constexpr (F == DT_Q4_K) {
                  isr[r] = __mul24(ksc[k], sl + sh);
                  msr[r] = __mul24(km[k], xg.sl + xg.sh);
                } else {
                  isr[r] = __mul24(ksc[k], sl - 32 * xg.sl) + __mul24(km[k], sh - 32 * xg.sh);
                }
              }
            }
            // exact integer sums over the 8 lanes of a super-block
            int rb;
            rows_sum8(isr, 8, rb);
            if constexpr (F == DT_Q4_K) rows_sum8(msr, 8, rb);
            const float dx = ((const float*)(xst + rb * RS + 32 * G))[gc];
            const double tt = superblock_q8k<F>(raw[k], isr[0], F == DT_Q4_K ? msr[0] : 0, dx);
            tot += (valid && g < G) ? tt : 0.0;
            base = rb;
          }
          if (lpr > 8) tot = tot + xswap<8>(tot);
          if (lpr > 16) tot = tot + xswap<16>(tot);
          if (lpr > 32) tot = tot + xswap<32>(tot);
          vr[0] = tot;
          n = 1;
        } else {
#pragma unroll
          for (int r = 0; r < RB; r++) {
            double accd = 0.0;
            if (r < nrows) {
#pragma unroll
              for (int k = 0; k < U; k++) {
                const int g = lr + k * lpr;
                XRow xg;
                stage_xrow<SUMS>(xst + r * RS, G, min(g, G - 1), xg);
                int sd = 0;
#pragma unroll
                for (int d = 0; d < 8; d++) sd = sdot4((int)cw[k][d], xg.w[d], sd);
                const double dxd = xg.dx;
                const int sxq = xg.sl + xg.sh;
                double tt;
                if constexpr (F == DT_Q8_0) {
                  tt = (double)sd * ((double)half_to_float(raw[k].a) * dxd);
                } else if constexpr (F == DT_MXFP4) {
                  tt = (double)sd * (mxfp4_q8_scale(raw[k].a) * dxd);
                } else if constexpr (F == DT_Q4_0) {
                  tt = (double)(sd - 8 * sxq) * ((double)half_to_float(raw[k].a) * dxd);
                } else if constexpr (F == DT_Q5_0) {
                  tt = (double)(sd - 16 * sxq) * ((double)half_to_float(raw[k].a) * dxd);
                } else {  // Q5_1
                  const double t1 = (double)sd * ((double)half_to_float(raw[k].a & 0xffffu) * dxd);
                  tt = t1 + (double)half_to_float(raw[k].a >> 16) * (dxd * (double)sxq);
                }
                if (valid && g < G) accd += tt;
              }
            }
            vr[r] = accd;
          }
          n = rows_sum8(vr, lpr, base);
        }
        if (lr < 8 && valid) {
#pragma unroll
          for (int i = 0; i < RB; i++) {
            if (i >= n) break;
            const int row = base + i;
            int64_t yo = yr[0];
#pragma unroll
            for (int r = 1; r < RB; r++) yo = row == r ? yr[r] : yo;
            double v = vr[i];
            if (bias) v = (double)bo + v;
            if (row < nrows) a.y[yo * a.out + o] = (float)v;
          }
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < RB; r++) {
        if (r >= nrows) break;
        const uint8_t* xrow = xst + r * RS;
        double v;
        if constexpr (is_k_quant(F)) {
          // the one-row GEMV's K-quant order: exact sums over the 8 lanes of
          // a super-block, the double term per lane, the super-block sets last
          int is[U], ms[U];
          XRow xg[U];
#pragma unroll
          for (int k = 0; k < U; k++) {
            const int g = lr + k * lpr;
            stage_xrow<SUMS>(xrow, G, min(g, G - 1), xg[k]);
            int sl = 0, sh = 0;
#pragma unroll
            for (int d = 0; d < 4; d++) {
              sl = sdot4((int)cw[k][d], xg[k].w[d], sl);
              sh = sdot4((int)cw[k][4 + d], xg[k].w[4 + d], sh);
            }
            if constexpr (F == DT_Q4_K) {
              is[k] = __mul24(ksc[k], sl + sh);
              ms[k] = __mul24(km[k], xg[k].sl + xg[k].sh);
            } else {
              is[k] = __mul24(ksc[k], sl - 32 * xg[k].sl) + __mul24(km[k], sh - 32 * xg[k].sh);
              ms[k] = 0;
            }
            const bool ok = valid && g < G;
            is[k] = ok ? is[k] : 0;
            ms[k] = ok ? ms[k] : 0;
          }
#pragma unroll
          for (int k = 0; k < U; k++) {
            is[k] = wave_sum(is[k], 8);
            ms[k] = wave_sum(ms[k], 8);
          }
          double tot = 0.0;
#pragma unroll
          for (int k = 0; k < U; k++) {
            const double tt = superblock_q8k<F>(raw[k], is[k], ms[k], xg[k].dx);
            tot += (valid && lr + k * lpr < G) ? tt : 0.0;
          }
          if (lpr > 8) tot = tot + xpart<8>(tot);
          if (lpr > 16) tot = tot + xpart<16>(tot);
          if (lpr > 32) tot = tot + xpart<32>(tot);
          v = tot;
        } else {
          double accd = 0.0;
#pragma unroll
          for (int k = 0; k < U; k++) {
            const int g = lr + k * lpr;
            XRow xg;
            stage_xrow<SUMS>(xrow, G, min(g, G - 1), xg);
            int sd = 0;
#pragma unroll
            for (int d = 0; d < 8; d++) sd = sdot4((int)cw[k][d], xg.w[d], sd);
            const double dxd = xg.dx;
            const int sxq = xg.sl + xg.sh;
            double tt;
            if constexpr (F == DT_Q8_0) {
              tt = (double)sd * ((double)half_to_float(raw[k].a) * dxd);
            } else if constexpr (F == DT_MXFP4) {
              tt = (double)sd * (mxfp4_q8_scale(raw[k].a) * dxd);
            } else if constexpr (F == DT_Q4_0) {
              tt = (double)(sd - 8 * sxq) * ((double)half_to_float(raw[k].a) * dxd);
            } else if constexpr (F == DT_Q5_0) {
              tt = (double)(sd - 16 * sxq) * ((double)half_to_float(raw[k].a) * dxd);
            } else {  // Q5_1
              const double t1 = (double)sd * ((double)half_to_float(raw[k].a & 0xffffu) * dxd);
              tt = t1 + (double)half_to_float(raw[k].a >> 16) * (dxd * (double)sxq);
            }
            if (valid && g < G) accd += tt;
          }
          v = wave_sum(accd, lpr);
        }
        if (lr == 0 && valid) {
          if (bias) v = (double)bo + v;
          a.y[yr[r] * a.out + o] = (float)v;
        }
      }
    }
    tb = nb;
#pragma unroll
    for (int i = 0; i < TB; i++)
#pragma unroll
      for (int k = 0; k < U; k++) cur[i][k] = nxt[i][k];
  }
}

// ------------------------------------------------------------ float rows
// One activation row against F32 / BF16 / F16 weights in the Q8 arithmetic
// (TInferCpuBackend.Linear's float branch, backend.cpu.pas:1548-1565: the
// exact float products summed in double). A wave takes one row per step;
// its 64 lanes read the row as consecutive 16-byte chunks (one contiguous
// kilobyte per load instruction), the next row's chunks in flight while this
// row is summed; the activation row is staged in LDS once per block (normed
// with NORM) and read per chunk. The rows of up to 3 matrices (nseg) are one
// index space, so the launch is one round of blocks whatever their shapes.
template <int F>
constexpr int f_bytes() { return F == DT_F32 ? 4 : 2; }

template <int F, bool NORM, int NJ>
__device__ __forceinline__ void gemv_flt(const LinArgs& a)
{
  constexpr int ES = f_bytes<F>(), VPC = 16 / ES;  // values per 16-byte chunk
  const int lane = threadIdx.x & 63;
  // the rows of the (up to 3) matrices as one index space: o0 rows of the
  // first, then o1 of the second, then o2 of the third; a wave takes every
  // nw-th of them (no block idles on a short matrix beside a long one)
  const int nseg = a.nseg > 1 ? a.nseg : 1;
  const int o0 = nseg > 1 ? a.oseg[0] : a.out, o1 = nseg > 1 ? a.oseg[1] : 0, o2 = nseg > 2 ? a.oseg[2] : 0;
  const int64_t total = (int64_t)o0 + o1 + o2;
  const int NC = a.in / VPC;  // chunks per row: at most 64 NJ
  const int nj = (NC + 63) / 64;
  const int64_t rb = (int64_t)a.in * ES;  // row bytes
  // with xq_out the launch's last block quantizes the normed row and takes
  // no rows (beside the row blocks, off their path)
  const bool qblock = NORM && a.xq_out && blockIdx.x == gridDim.x - 1;
  const int64_t nw = (int64_t)(gridDim.x - (NORM && a.xq_out ? 1 : 0)) * (NT >> 6);
  const int64_t wid = (int64_t)blockIdx.x * (NT >> 6) + (threadIdx.x >> 6);
  __shared__ __align__(16) float xs[XN];
  if (!qblock && (int64_t)blockIdx.x * (NT >> 6) >= total) return;  // the whole block: no rows
  // (selected, not indexed: an index into the argument block would move it
  // to scratch memory)
  auto wrow = [&](int64_t g, int& sg, int& o) -> const uint8_t* {
    sg = g < o0 ? 0 : (g < (int64_t)o0 + o1 ? 1 : 2);
    o = (int)(g - (sg == 0 ? 0 : (sg == 1 ? o0 : (int64_t)o0 + o1)));
    const uint8_t* w = nseg > 1 ? (sg == 0 ? a.wseg[0] : (sg == 1 ? a.wseg[1] : a.wseg[2])) : a.w;
    return w + (int64_t)o * rb;
  };
  auto load = [&](int64_t g, uint4 (&wv)[NJ]) {
    int sg, o;
    const uint8_t* wr = wrow(min(g, total - 1), sg, o);
#pragma unroll
    for (int j = 0; j < NJ; j++)
      if (j < nj) {  // the same for the whole launch
        const int c = min(lane + 64 * j, NC - 1);
        wv[j] = ld<uint4, true>(wr, (uint32_t)c * 16u);
      }
  };
  XStage st;
  stage_load<F, 1, NORM>(a.x, nullptr, a.in, a.nw, st);
  // the first row's weights while the activation row is staged
  uint4 wv[NJ], wn[NJ];
  int64_t g = wid;
  load(g, wv);
  stage_store<F, 1, NORM>(st, false, a.in, a.eps, (uint8_t*)xs, nullptr, a.bad, 1);
  __syncthreads();
  if constexpr (NORM) {
    // the normed row quantized for the next launch: wave w of the last block
    // takes 64 quarters (2 super-blocks, 16 groups) at a time, from quarter
    // 64 w on
    if (qblock) {
      const int nq = a.in >> 3;
      for (int q0 = (int)(threadIdx.x >> 6) * 64; q0 < nq; q0 += 256) {
        const int q = q0 + lane;
        float v[8];
        const float4 u0 = ((const float4*)xs)[2 * min(q, nq - 1)], u1 = ((const float4*)xs)[2 * min(q, nq - 1) + 1];
        v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
        v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
        uint32_t c0, c1;
        float dx;
        bool nonfinite;
        if (a.xq_k8) quant_quarter<true>(v, q, c0, c1, dx, nonfinite);
        else quant_quarter<false>(v, q, c0, c1, dx, nonfinite);
        if (q < nq) {
          ((uint2*)a.xq_out)[q] = make_uint2(c0, c1);
          if ((q & 3) == 0) ((float*)(a.xq_out + a.in))[q >> 2] = dx;
          if (nonfinite && a.bad) a.bad[0] = 1;
        }
      }
      return;
    }
  }
  while (g < total) {
    // the next row's weights in flight during this row's sums
    const int64_t gn = g + nw;
    if (gn < total) load(gn, wn);
    double p[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int c = lane + 64 * j;
      if (j < nj && c < NC) {
        const uint32_t q[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          if constexpr (F == DT_F32) {
            v[i] = bits_float(q[i]);
          } else if constexpr (F == DT_BF16) {
            v[2 * i] = bits_float(q[i] << 16);
            v[2 * i + 1] = bits_float(q[i] & 0xffff0000u);
          } else {
            v[2 * i] = half_to_float(q[i] & 0xffffu);
            v[2 * i + 1] = half_to_float(q[i] >> 16);
          }
        }
        const float4* xp = (const float4*)(xs + c * VPC);
#pragma unroll
        for (int h = 0; h < VPC / 4; h++) {
          const float4 xv = xp[h];
          p[0] = __builtin_fma((double)v[4 * h], (double)xv.x, p[0]);
          p[1] = __builtin_fma((double)v[4 * h + 1], (double)xv.y, p[1]);
          p[2] = __builtin_fma((double)v[4 * h + 2], (double)xv.z, p[2]);
          p[3] = __builtin_fma((double)v[4 * h + 3], (double)xv.w, p[3]);
        }
      }
    }
    double v = wave_sum((p[0] + p[1]) + (p[2] + p[3]), 64);
    if (lane == 0) {
      int sg, o;
      (void)wrow(g, sg, o);
      const float* bias = nseg > 1 ? (sg == 0 ? a.bseg[0] : (sg == 1 ? a.bseg[1] : a.bseg[2])) : a.bias;
      float* yp = nseg > 1 ? (sg == 0 ? a.yseg[0] : (sg == 1 ? a.yseg[1] : a.yseg[2])) : a.y;
      if (bias) v = (double)bias[o] + v;
      float rr = (float)v;
      if (a.res) rr = a.res[o] + rr;
      yp[o] = rr;
    }
    g = gn;
#pragma unroll
    for (int j = 0; j < NJ; j++) wv[j] = wn[j];
  }
}

// ------------------------------------------------------------------ combine
// The down projection of one token's experts, added into the residual:
// TDecoderModel.Experts (decoder.pas:3140-3148) - every expert row as a float
// (its bias added in double first), then the rows weighted by cw and summed
// in slot order, each step single-rounded, then added to the residual.
// A block of 4 waves takes one tile of rows per step; wave w computes slots
// w and w + 4 (kslots <= 8), the values meet in LDS and wave 0 adds them in
// slot order. The kslots activation rows x[s] (contiguous) are staged once
// per block into the dynamic LDS.
template <int F, int MODE, int U>
__device__ __forceinline__ void gemv_cmb(const LinArgs& a)
{
  extern __shared__ __align__(16) uint8_t cmb_xs[];
  __shared__ float dv[8][8];  // [slot][row of the tile]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = a.lpr, lr = lane & (lpr - 1), rsub = lane / lpr, rpw = 64 / lpr;
  const int G = a.in >> 5, K = a.kslots;
  const Regions rg = regions(F, a.out, a.in);
  const int64_t tiles = ((int64_t)a.out + rpw - 1) / rpw;
  const int n = K * a.in;
  float* dxs = (float*)(cmb_xs + n);
  // the activation rows need no expert id: their loads go first (the first
  // XN values; more, gpt-oss's 4 x 2880, in further chunks below)
  IHIP_STAMP_SCOPE;
  IHIP_STAMP(0);
  const int nc0 = min(XN, n);
  XStage st0;
  stage_load<F, MODE, false>(a.x, nullptr, nc0, nullptr, st0);
  IHIP_STAMP(6);
  // this wave's slots and their experts (a bad id adds nothing)
  const uint8_t* wi[2];
  bool ok[2];
  int64_t e[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int sl = wave + 4 * i;
    const int id = sl < K ? a.ids[sl] : -1;
    ok[i] = sl < K && id >= 0 && (a.nexp <= 0 || id < a.nexp);
    e[i] = ok[i] ? id : 0;
    wi[i] = a.w + e[i] * a.stride;
  }
  Raw raw[2][U];
  float eb[2], er;  // the tile row's expert biases and residual, loaded with its weights
  int64_t t = blockIdx.x;
  auto load = [&](int64_t tt) {
    const int64_t o = min(tt * rpw + rsub, (int64_t)a.out - 1);
    if constexpr (!is_float_type(F)) {
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int k = 0; k < U; k++)
          load_group<F, true, F == DT_Q4_K>(wi[i], rg, o, G, min(lr + k * lpr, G - 1), a.in, raw[i][k]);
    }
    // (a launch without them issues no load for them: a uniform branch)
#pragma unroll
    for (int i = 0; i < 2; i++) eb[i] = a.bias ? a.bias[e[i] * a.out + o] : 0.f;
    er = a.res ? a.res[o] : 0.f;
  };
  load(t);
  IHIP_STAMP(1);
  stage_store<F, MODE, false>(st0, false, nc0, 0.0, cmb_xs, dxs, a.bad, 1);
  for (int c0 = XN; c0 < n; c0 += XN) {
    XStage st;
    const int nc = min(XN, n - c0);
    stage_load<F, MODE, false>(a.x + c0, nullptr, nc, nullptr, st);
    stage_store<F, MODE, false>(st, false, nc, 0.0,
                         cmb_xs + (stage_q8<F, MODE>() ? c0 : 4 * c0), dxs + c0 / 32, a.bad, 1);
  }
  __syncthreads();
  IHIP_STAMP(2);
  while (t < tiles) {
    const int64_t o = t * rpw + rsub;
    const bool valid = o < a.out;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int sl = wave + 4 * i;
      if (sl < K) {  // the same for the whole wave
        XGroup xg[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
          const int g = lr + k * lpr;
          xg[k] = XGroup{};
          if (g < G) lds_x<F, MODE>(cmb_xs, dxs, sl * G + g, xg[k]);
        }
        double v = row_value<F, MODE, U>(wi[i], raw[i], o, valid && ok[i], xg, lr, lpr, G, a.in);
        if (lr == 0) {
          float d = 0.f;
          if (valid && ok[i]) {
            if (a.bias) v = (double)eb[i] + v;
            d = (float)v;
          }
          dv[sl][rsub] = d;
        }
      }
    }
    __syncthreads();
    IHIP_STAMP(4);
    const float res = er;  // this tile's residual, before the next tile's loads
    const int64_t tn = t + gridDim.x;
    if (tn < tiles) load(tn);
    if (wave == 0 && lr == 0 && valid) {
      float add = 0.f;
      for (int sl = 0; sl < K; sl++) {
        float p = a.cw[sl] * dv[sl][rsub];
        add = add + p;
      }
      a.y[o] = a.res ? res + add : add;
    }
    __syncthreads();
    t = tn;
  }
  IHIP_STAMP(5);
}

// ------------------------------------------------------------ dequant/embed
// y[r] = InferRowToF32 of row (ids ? ids[r] : row0 + r), bit-exact: every
// value formed as tensor.pas:467-602 forms it. One wave per row, one group
// per lane step.
struct DeqArgs {
  const uint8_t* w;
  const int* ids;
  float* y;
  int64_t row0;
  int32_t out, in, rows, pad;
};

template <int F>
__device__ __forceinline__ void dequant(const DeqArgs& a)
{
  int wrow = blockIdx.x * (NT >> 6) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (wrow >= a.rows) return;
  int64_t o = a.ids ? (int64_t)a.ids[wrow] : a.row0 + wrow;
  int G = a.in >> 5;
  if (o < 0 || o >= a.out) {  // an id outside the table: a zero row
    for (int c = lane; c < a.in; c += 64) a.y[(int64_t)wrow * a.in + c] = 0.f;
    return;
  }
  const Regions rg = regions(F, a.out, a.in);
  float* yr = a.y + (int64_t)wrow * a.in;
  for (int g = lane; g < G; g += 64) {
    float v[32];
    if constexpr (is_float_type(F)) {
      load_fgroup<F>(a.w, o, g, a.in, v);
    } else {
      Raw r;
      load_group<F, true>(a.w, rg, o, G, g, a.in, r);
#pragma unroll
      for (int hi = 0; hi < 2; hi++)
#pragma unroll
        for (int d = 0; d < 4; d++) {
          uint32_t c = code_bytes<F>(r, d, hi);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            int j = 16 * hi + 4 * d + i;
            uint32_t u = (c >> (8 * i)) & 255u;
            float val;
            if constexpr (F == DT_Q8_0) {
              val = half_to_float(r.a) * (float)(int)(int8_t)u;
            } else if constexpr (F == DT_MXFP4) {
              val = e8m0_half(r.a) * (float)(int)(int8_t)u;
            } else if constexpr (F == DT_Q4_0) {
              val = half_to_float(r.a) * (float)((int)u - 8);
            } else if constexpr (F == DT_Q5_0) {
              val = half_to_float(r.a) * (float)((int)u - 16);
            } else if constexpr (F == DT_Q5_1) {
              float t = half_to_float(r.a & 0xffffu) * (float)u;
              val = t + half_to_float(r.a >> 16);
            } else if constexpr (F == DT_Q4_K) {
              int sc, m;
              scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, m);
              float d1 = half_to_float(r.q1.x & 0xffffu) * (float)sc;
              float m1 = half_to_float(r.q1.x >> 16) * (float)m;
              float t = d1 * (float)u;
              val = t - m1;
            } else {  // Q6_K
              float t = half_to_float(r.d) * (float)(int)(int8_t)(hi ? (r.a >> 8) : (r.a & 255u));
              val = t * (float)((int)u - 32);
            }
            v[j] = val;
          }
        }
    }
    float4* p = (float4*)(yr + (int64_t)g * 32);
#pragma unroll
    for (int k = 0; k < 8; k++) p[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  }
}

}  // namespace ihip

// ------------------------------------------------------- exported symbols
#define IHIP_GEMV(NAME, F, M, U, R, GLU, ...) \
  extern "C" __global__ __launch_bounds__(256) void NAME(ihip::LinArgs a) { ihip::touch_kernargs<sizeof(ihip::LinArgs)>(); ihip::gemv<F, M, U, R, GLU, __VA_ARGS__>(a); }

#define IHIP_GEMV_U(PFX, F, M)                       \
  IHIP_GEMV(PFX##_u1, F, M, 1, 1, false, false)      \
  IHIP_GEMV(PFX##_u2, F, M, 2, 1, false, false)      \
  IHIP_GEMV(PFX##_u3, F, M, 3, 1, false, false)      \
  IHIP_GEMV(PFX##_u4, F, M, 4, 1, false, false)      \
  IHIP_GEMV(PFX##_glu_u1, F, M, 1, 1, true, false)   \
  IHIP_GEMV(PFX##_glu_u2, F, M, 2, 1, true, false)   \
  IHIP_GEMV(PFX##_glu_u3, F, M, 3, 1, true, false)   \
  IHIP_GEMV(PFX##_glu_u4, F, M, 4, 1, true, false)   \
  IHIP_GEMV(PFX##_norm_u1, F, M, 1, 1, false, true)  \
  IHIP_GEMV(PFX##_norm_u2, F, M, 2, 1, false, true)  \
  IHIP_GEMV(PFX##_norm_u3, F, M, 3, 1, false, true)  \
  IHIP_GEMV(PFX##_norm_u4, F, M, 4, 1, false, true)  \
  IHIP_GEMV(PFX##_norm_glu_u1, F, M, 1, 1, true, true) \
  IHIP_GEMV(PFX##_norm_glu_u2, F, M, 2, 1, true, true) \
  IHIP_GEMV(PFX##_norm_glu_u3, F, M, 3, 1, true, true) \
  IHIP_GEMV(PFX##_norm_glu_u4, F, M, 4, 1, true, true) \
  IHIP_GEMV(PFX##_b8u1, F, M, 1, 8, false, false)    \
  IHIP_GEMV(PFX##_b8u2, F, M, 2, 8, false, false)    \
  IHIP_GEMV(PFX##_b8u3, F, M, 3, 8, false, false)    \
  IHIP_GEMV(PFX##_b8u4, F, M, 4, 8, false, false)

#define IHIP_ROWS(NAME, F, U, TB) \
  extern "C" __global__ __launch_bounds__(256) void NAME(ihip::LinArgs a) { ihip::touch_kernargs<sizeof(ihip::LinArgs)>(); ihip::gemv_rows<F, U, TB>(a); }
#define IHIP_ROWS_U(PFX, F)         \
  IHIP_ROWS(PFX##_r8u1, F, 1, 2)    \
  IHIP_ROWS(PFX##_r8u2, F, 2, 1)    \
  IHIP_ROWS(PFX##_r8u3, F, 3, 1)    \
  IHIP_ROWS(PFX##_r8u4, F, 4, 1)

#define IHIP_CMB(NAME, F, M, U) \
  extern "C" __global__ __launch_bounds__(256) void NAME(ihip::LinArgs a) { ihip::touch_kernargs<sizeof(ihip::LinArgs)>(); ihip::gemv_cmb<F, M, U>(a); }

#define IHIP_CMB_U(PFX, F, M)      \
  IHIP_CMB(PFX##_cmb_u1, F, M, 1) \
  IHIP_CMB(PFX##_cmb_u2, F, M, 2) \
  IHIP_CMB(PFX##_cmb_u3, F, M, 3) \
  IHIP_CMB(PFX##_cmb_u4, F, M, 4)

// q, k and v of a Q4_K_M model in one launch: Q4_K matrices, then Q6_K ones
#define IHIP_GEMV_MIX(NAME, F, F2, M, U)                                              \
  extern "C" __global__ __launch_bounds__(256) void NAME(ihip::LinArgs a)               \
  {                                                                                    \
    ihip::touch_kernargs<sizeof(ihip::LinArgs)>();                                     \
    if (ihip::seg_of(a) < a.nseg1) ihip::gemv<F, M, U, 1, false, true>(a);             \
    else ihip::gemv<F2, M, U, 1, false, true>(a);                                      \
  }
#define IHIP_GEMV_MIX_U(PFX, F, F2, M) \
  IHIP_GEMV_MIX(PFX##_norm_u1, F, F2, M, 1) IHIP_GEMV_MIX(PFX##_norm_u2, F, F2, M, 2) \
  IHIP_GEMV_MIX(PFX##_norm_u3, F, F2, M, 3) IHIP_GEMV_MIX(PFX##_norm_u4, F, F2, M, 4)

#define IHIP_FLT1(NAME, F, NORM, NJ)                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(ihip::LinArgs a)       \
  {                                                                             \
    ihip::touch_kernargs<sizeof(ihip::LinArgs)>();                              \
    ihip::gemv_flt<F, NORM, NJ>(a);                                             \
  }
// rows of at most 512 (j8) or 1024 (j16) 16-byte chunks
#define IHIP_FLT(NAME, F)                                       \
  IHIP_FLT1(gemv_##NAME##_q8_rows_j8, F, false, 8)              \
  IHIP_FLT1(gemv_##NAME##_q8_rows_j16, F, false, 16)            \
  IHIP_FLT1(gemv_##NAME##_q8_norm_rows_j8, F, true, 8)          \
  IHIP_FLT1(gemv_##NAME##_q8_norm_rows_j16, F, true, 16)

#define IHIP_GEMV_FMT(NAME, F) \
  IHIP_GEMV_U(gemv_##NAME##_f32, F, 0) \
  IHIP_GEMV_U(gemv_##NAME##_q8, F, 1) \
  IHIP_CMB_U(gemv_##NAME##_f32, F, 0) \
  IHIP_CMB_U(gemv_##NAME##_q8, F, 1)

#define IHIP_DEQ(NAME, F) \
  extern "C" __global__ __launch_bounds__(256) void dequant_##NAME(ihip::DeqArgs a) { ihip::dequant<F>(a); }
#ifdef IHIP_ONLY_FMT_Q8_0
IHIP_GEMV_FMT(q8_0, ihip::DT_Q8_0)
IHIP_ROWS_U(gemv_q8_0_q8, ihip::DT_Q8_0)
IHIP_DEQ(q8_0, ihip::DT_Q8_0)
#endif
#ifdef IHIP_ONLY_FMT_Q4_0
IHIP_GEMV_FMT(q4_0, ihip::DT_Q4_0)
IHIP_ROWS_U(gemv_q4_0_q8, ihip::DT_Q4_0)
IHIP_DEQ(q4_0, ihip::DT_Q4_0)
#endif
#ifdef IHIP_ONLY_FMT_MXFP4
IHIP_GEMV_FMT(mxfp4, ihip::DT_MXFP4)
IHIP_ROWS_U(gemv_mxfp4_q8, ihip::DT_MXFP4)
IHIP_DEQ(mxfp4, ihip::DT_MXFP4)
#endif
#ifdef IHIP_ONLY_FMT_Q5_0
IHIP_GEMV_FMT(q5_0, ihip::DT_Q5_0)
IHIP_ROWS_U(gemv_q5_0_q8, ihip::DT_Q5_0)
IHIP_DEQ(q5_0, ihip::DT_Q5_0)
#endif
#ifdef IHIP_ONLY_FMT_Q5_1
IHIP_GEMV_FMT(q5_1, ihip::DT_Q5_1)
IHIP_ROWS_U(gemv_q5_1_q8, ihip::DT_Q5_1)
IHIP_DEQ(q5_1, ihip::DT_Q5_1)
#endif
#ifdef IHIP_ONLY_FMT_Q4_K
IHIP_GEMV_FMT(q4_k, ihip::DT_Q4_K)
IHIP_ROWS_U(gemv_q4_k_q8, ihip::DT_Q4_K)
IHIP_GEMV_MIX_U(gemv_q4_k_q6_k_q8, ihip::DT_Q4_K, ihip::DT_Q6_K, 1)
IHIP_GEMV_MIX_U(gemv_q4_k_q6_k_f32, ihip::DT_Q4_K, ihip::DT_Q6_K, 0)
IHIP_DEQ(q4_k, ihip::DT_Q4_K)
#endif
#ifdef IHIP_ONLY_FMT_Q6_K
IHIP_GEMV_FMT(q6_k, ihip::DT_Q6_K)
IHIP_ROWS_U(gemv_q6_k_q8, ihip::DT_Q6_K)
IHIP_DEQ(q6_k, ihip::DT_Q6_K)
#endif
#ifdef IHIP_ONLY_FMT_F32
IHIP_GEMV_FMT(f32, ihip::DT_F32)
IHIP_FLT(f32, ihip::DT_F32)
IHIP_DEQ(f32, ihip::DT_F32)
#endif
#ifdef IHIP_ONLY_FMT_BF16
IHIP_GEMV_FMT(bf16, ihip::DT_BF16)
IHIP_FLT(bf16, ihip::DT_BF16)
IHIP_DEQ(bf16, ihip::DT_BF16)
#endif
#ifdef IHIP_ONLY_FMT_F16
IHIP_GEMV_FMT(f16, ihip::DT_F16)
IHIP_FLT(f16, ihip::DT_F16)
IHIP_DEQ(f16, ihip::DT_F16)
#endif
