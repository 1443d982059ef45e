// gemm.hip - the prefill GEMM of the Q8 arithmetic on the int8 matrix cores
// of gfx950 (one weight type per build, IHIP_ONLY_FMT_*).
//
// What it computes: y[r, o] = bias[o] + sum over groups of the exact
// TInferCpuBackend.Linear terms (backend.cpu.pas:1409-1566, 823-967) for
// quantized activation rows x (Q8_0 or Q8_K, by quantize_q8_0/_k) and weights
// in the HIP layout of layout.h - the same terms, in double, as the one-row
// GEMV of linear.hip (group_q8, group_q8k, superblock_q8k); only the order of
// the double sum over groups differs (here: group order).
//
// Mapping to CDNA4: a block of 4 waves owns 64 rows x 64 outputs, each wave
// 32 x 32. Per 32-value group a wave runs v_mfma_i32_32x32x32_i8 with A = the
// activation codes of its 32 rows and B = the weight codes of its 32
// outputs, widened to int8 (centred for Q4_0/Q5_0/Q6_K, the e2m1 table for
// MXFP4): the exact int32 group dot products, 16 per lane. The lanes then
// apply the scales in double: a lane owns one output (its scales are
// per-lane registers) and 16 rows (their activation scales and code sums are
// staged in LDS per 8 groups). Q6_K's 16-value sub-blocks are two
// v_mfma_i32_32x32x16_i8, lane half h feeding values 8h..8h+7 of each
// sub-block: with the group's nibble order (byte j: value j, value j + 16)
// both come from bytes 8h..8h+7 of the 16-byte group.
//
// Operand layout of both MFMAs (probed on gfx950): A lane l = row l % 32,
// B lane l = column l % 32, 16 (8) k values each, the k order free but the
// same in A and B; result register i of lane l = row 8 (i / 4) + 4 (l / 32) +
// i % 4, column l % 32.
#include "formats.h"

namespace ihip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const uint8_t* w;   // matrix, or expert 0 with items
  const uint8_t* xq;  // quantized rows [*, in + 4 G]: int8 codes, then float dx per group
  const float* bias;  // [out], [experts, out] with items, or null
  float* y;           // [*, out]
  int64_t stride;     // bytes between experts
  int32_t out, in, rows, pad;
  // grouped experts: tile row block blockIdx.y = item (expert, start, count
  // <= 64) over perm, the slots sorted by expert; slot s reads x row
  // s / x_per_slot (0: row 0) and writes y row s
  const int4* items;
  const int* perm;
  int32_t x_per_slot, pad2;
};

constexpr int GBM = 64, GBN = 64, GKC = 8;  // tile rows, outputs, groups per LDS stage

// the weight codes of lane half h (values 8h..8h+7 and 16+8h..16+8h+7 of the
// group) as 16 int8 in the Q8 arithmetic's value (centred where the format
// has an offset the CPU subtracts through the activation sum)
template <int F>
__device__ __forceinline__ v4i b_operand(const Raw& r, int h)
{
  uint32_t c[4] = {code_bytes<F>(r, 2 * h, 0), code_bytes<F>(r, 2 * h + 1, 0),
                   code_bytes<F>(r, 2 * h, 1), code_bytes<F>(r, 2 * h + 1, 1)};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    uint32_t t = c[k];
    if constexpr (F == DT_Q4_0) {  // q - 8: the 4-bit value sign-extended after flipping bit 3
      t ^= 0x08080808u;
      t |= (t & 0x08080808u) * 0x1Eu;
    } else if constexpr (F == DT_Q5_0) {  // q - 16
      t ^= 0x10101010u;
      t |= (t & 0x10101010u) * 0x0Eu;
    } else if constexpr (F == DT_Q6_K) {  // q - 32
      t ^= 0x20202020u;
      t |= (t & 0x20202020u) * 0x06u;
    }
    c[k] = t;
  }
  return v4i{(int)c[0], (int)c[1], (int)c[2], (int)c[3]};
}

// does the format need the activation code sum of a group (through the
// minimum / offset the CPU applies with it)
constexpr bool needs_xsum(int F) { return F == DT_Q4_K || F == DT_Q5_1; }

template <int F>
__device__ __forceinline__ void gemm(const GemmArgs& a)
{
  __shared__ float sdx[GKC][GBM];  // activation scales of the chunk's groups
  __shared__ int sbs[GKC][GBM];    // activation code sums (Q4_K, Q5_1)
  __shared__ int sxr[GBM], syr[GBM];
  const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5;
  const int wm = w & 1, wn = w >> 1;
  const int G = a.in >> 5;
  const int64_t xstride = (int64_t)a.in + 4 * (int64_t)G;
  const uint8_t* wb = a.w;
  const float* bias = a.bias;
  int nrows;
  if (a.items) {
    const int4 it = a.items[blockIdx.y];
    if (it.z <= 0) return;
    wb += (int64_t)it.x * a.stride;
    if (bias) bias += (int64_t)it.x * a.out;
    nrows = min(GBM, it.z);
    if (t < GBM) {
      const int sl = a.perm[it.y + min(t, nrows - 1)];
      sxr[t] = a.x_per_slot ? sl / a.x_per_slot : 0;
      syr[t] = sl;
    }
  } else {
    const int r0 = blockIdx.y * GBM;
    nrows = min(GBM, a.rows - r0);
    if (t < GBM) sxr[t] = syr[t] = r0 + min(t, nrows - 1);
  }
  __syncthreads();
  const Regions rg = regions(F, a.out, a.in);
  const int o_real = blockIdx.x * GBN + 32 * wn + (l & 31);
  const int64_t o = min(o_real, a.out - 1);
  const uint8_t* xa = a.xq + (int64_t)sxr[32 * wm + (l & 31)] * xstride;  // this lane's A row
  const int rb = 32 * wm + 4 * h;  // tile row of result register i: rb + 8 (i / 4) + i % 4

  double acc[16];
  int isum[16], msum[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    acc[i] = 0.0;
    isum[i] = msum[i] = 0;
  }

  for (int gc = 0; gc < G; gc += GKC) {
    __syncthreads();  // the previous chunk's LDS reads are done
    for (int e = t; e < GKC * GBM; e += 256) {
      const int j = e / GBM, rt = e % GBM, g = min(gc + j, G - 1);
      const uint8_t* xr = a.xq + (int64_t)sxr[rt] * xstride;
      sdx[j][rt] = ((const float*)(xr + a.in))[g];
      if constexpr (needs_xsum(F)) {
        const uint4* p = (const uint4*)(xr + (int64_t)g * 32);
        uint4 u0 = p[0], u1 = p[1];
        int sm = 0;
        sm = sdot4((int)u0.x, 0x01010101, sm); sm = sdot4((int)u0.y, 0x01010101, sm);
        sm = sdot4((int)u0.z, 0x01010101, sm); sm = sdot4((int)u0.w, 0x01010101, sm);
        sm = sdot4((int)u1.x, 0x01010101, sm); sm = sdot4((int)u1.y, 0x01010101, sm);
        sm = sdot4((int)u1.z, 0x01010101, sm); sm = sdot4((int)u1.w, 0x01010101, sm);
        sbs[j][rt] = sm;
      }
    }
    __syncthreads();
    const int nj = min(GKC, G - gc);
    for (int j = 0; j < nj; j++) {
      const int g = gc + j;
      Raw r;
      load_group<F>(wb, rg, o, G, g, a.in, r);
      const uint2 x0 = *(const uint2*)(xa + (int64_t)g * 32 + 8 * h);
      const uint2 x1 = *(const uint2*)(xa + (int64_t)g * 32 + 16 + 8 * h);
      const v4i bv = b_operand<F>(r, h);
      v16i s;
      v16i s2 = {};
      if constexpr (F == DT_Q6_K) {
        // the two 16-value sub-blocks of the group, each its own sum
        const v16i z = {};
        s = __builtin_amdgcn_mfma_i32_32x32x16_i8(
            (long)(((uint64_t)x0.y << 32) | x0.x),
            (long)(((uint64_t)(uint32_t)bv.y << 32) | (uint32_t)bv.x), z, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_i32_32x32x16_i8(
            (long)(((uint64_t)x1.y << 32) | x1.x),
            (long)(((uint64_t)(uint32_t)bv.w << 32) | (uint32_t)bv.z), z, 0, 0, 0);
      } else {
        const v4i av = {(int)x0.x, (int)x0.y, (int)x1.x, (int)x1.y};
        const v16i z = {};
        s = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, z, 0, 0, 0);
      }
      // the group's terms (group_q8 / group_q8k / superblock_q8k)
      if constexpr (F == DT_Q4_K) {
        int sc, mn;
        scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, mn);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          isum[i] += sc * s[i];
          msum[i] += mn * sbs[j][rb + 8 * (i >> 2) + (i & 3)];
        }
        if ((g & 7) == 7) {
          const double hd = half_to_float(r.q1.x & 0xffffu), hm = half_to_float(r.q1.x >> 16);
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const double dx = sdx[j][rb + 8 * (i >> 2) + (i & 3)];
            acc[i] = acc[i] + ((hd * dx) * (double)isum[i] - (hm * dx) * (double)msum[i]);
            isum[i] = msum[i] = 0;
          }
        }
      } else if constexpr (F == DT_Q6_K) {
        const int sa = (int)(int8_t)(r.a & 255u), sb = (int)(int8_t)(r.a >> 8);
#pragma unroll
        for (int i = 0; i < 16; i++) isum[i] += sa * s[i] + sb * s2[i];
        if ((g & 7) == 7) {
          const double d = half_to_float(r.d);
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const double dx = sdx[j][rb + 8 * (i >> 2) + (i & 3)];
            acc[i] = acc[i] + (d * dx) * (double)isum[i];
            isum[i] = 0;
          }
        }
      } else if constexpr (F == DT_Q5_1) {
        const double d = half_to_float(r.a & 0xffffu), m = half_to_float(r.a >> 16);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int ri = rb + 8 * (i >> 2) + (i & 3);
          const double dx = sdx[j][ri];
          const double tt = (double)s[i] * (d * dx);
          acc[i] = acc[i] + (tt + m * (dx * (double)sbs[j][ri]));
        }
      } else {
        double dw;
        if constexpr (F == DT_MXFP4) dw = mxfp4_q8_scale(r.a);
        else dw = half_to_float(r.a);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const double dx = sdx[j][rb + 8 * (i >> 2) + (i & 3)];
          acc[i] = acc[i] + ((double)s[i] * dw) * dx;
        }
      }
    }
  }
  if (o_real >= a.out) return;
  const double b = bias ? (double)bias[o] : 0.0;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int rt = rb + 8 * (i >> 2) + (i & 3);
    if (rt < nrows) {
      double v = acc[i];
      if (bias) v = b + v;
      a.y[(int64_t)syr[rt] * a.out + o] = (float)v;
    }
  }
}

}  // namespace ihip

#define IHIP_GEMM(NAME, F) \
  extern "C" __global__ __launch_bounds__(256) void gemm_##NAME(ihip::GemmArgs a) { ihip::gemm<F>(a); }

#ifdef IHIP_ONLY_FMT_Q8_0
IHIP_GEMM(q8_0, ihip::DT_Q8_0)
#endif
#ifdef IHIP_ONLY_FMT_Q4_0
IHIP_GEMM(q4_0, ihip::DT_Q4_0)
#endif
#ifdef IHIP_ONLY_FMT_MXFP4
IHIP_GEMM(mxfp4, ihip::DT_MXFP4)
#endif
#ifdef IHIP_ONLY_FMT_Q5_0
IHIP_GEMM(q5_0, ihip::DT_Q5_0)
#endif
#ifdef IHIP_ONLY_FMT_Q5_1
IHIP_GEMM(q5_1, ihip::DT_Q5_1)
#endif
#ifdef IHIP_ONLY_FMT_Q4_K
IHIP_GEMM(q4_k, ihip::DT_Q4_K)
#endif
#ifdef IHIP_ONLY_FMT_Q6_K
IHIP_GEMM(q6_k, ihip::DT_Q6_K)
#endif
