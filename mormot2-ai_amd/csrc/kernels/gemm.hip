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
  const float* x;  // float rows [*, in] (float weights)
  // float weights, ksplit > 1: block z sums the values [z klen, (z + 1) klen)
  // and writes its double partial sums (no bias) to part [ksplit, rows, out]
  double* part;
  int32_t ksplit, klen;
};

constexpr int GBM = 64, GBN = 64, GKC = 8;  // tile rows, outputs, groups per chunk

// the weight codes of lane half h (values 8h..8h+7 and 16+8h..16+8h+7 of the
// group) as 16 int8 in the Q8 arithmetic's value (centred where the format
// has an offset the CPU subtracts through the activation sum)
template <int F>
__device__ __forceinline__ v4i b_operand(const Raw& r, int h)
{
  // the lane half's view of the group: code dwords 2h and 2h + 1 moved to
  // dwords 0 and 1, chosen by masks (values, never an index into registers)
  const uint32_t m = 0u - (uint32_t)h;
  Raw v = r;
  v.q0.x = (r.q0.x & ~m) | (r.q0.z & m);
  v.q0.y = (r.q0.y & ~m) | (r.q0.w & m);
  v.q1.x = (r.q1.x & ~m) | (r.q1.z & m);
  v.q1.y = (r.q1.y & ~m) | (r.q1.w & m);
  if constexpr (F == DT_Q5_0 || F == DT_Q5_1) v.b = r.b >> (8 * h);  // 4 bits per code dword
  if constexpr (F == DT_Q6_K) {  // 2 bits per code dword
    v.b = r.b >> (4 * h);
    v.c = r.c >> (4 * h);
  }
  uint32_t c[4] = {code_bytes<F>(v, 0, 0), code_bytes<F>(v, 1, 0), code_bytes<F>(v, 0, 1),
                   code_bytes<F>(v, 1, 1)};
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

// The fields of Raw a format uses, as dwords: how a weight group sits in LDS.
template <int F>
constexpr int raw_dwords()
{
  return F == DT_Q8_0 ? 9 : (F == DT_Q4_K || F == DT_Q6_K) ? 8 : (F == DT_Q5_0 || F == DT_Q5_1) ? 6 : 5;
}

template <int F>
__device__ __forceinline__ void raw_put(uint32_t* d, int stride, const Raw& r)
{
  uint32_t v[9] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, 0, 0, 0, 0, 0};
  if constexpr (F == DT_Q8_0 || F == DT_Q4_K) {
    v[4] = r.q1.x; v[5] = r.q1.y; v[6] = r.q1.z; v[7] = r.q1.w;
    v[8] = r.a;
  } else if constexpr (F == DT_Q6_K) {
    v[4] = r.a; v[5] = r.b; v[6] = r.c; v[7] = r.d;
  } else {
    v[4] = r.a;
    v[5] = r.b;
  }
#pragma unroll
  for (int k = 0; k < raw_dwords<F>(); k++) d[k * stride] = v[k];
}

template <int F>
__device__ __forceinline__ Raw raw_get(const uint32_t* d, int stride)
{
  uint32_t v[9];
#pragma unroll
  for (int k = 0; k < raw_dwords<F>(); k++) v[k] = d[k * stride];
  Raw r{};
  r.q0 = make_uint4(v[0], v[1], v[2], v[3]);
  if constexpr (F == DT_Q8_0 || F == DT_Q4_K) {
    r.q1 = make_uint4(v[4], v[5], v[6], v[7]);
    if constexpr (F == DT_Q8_0) r.a = v[8];
  } else if constexpr (F == DT_Q6_K) {
    r.a = v[4]; r.b = v[5]; r.c = v[6]; r.d = v[7];
  } else {
    r.a = v[4];
    if constexpr (F == DT_Q5_0 || F == DT_Q5_1) r.b = v[5];
  }
  return r;
}

// A chunk of GKC groups of a block's tile, loaded cooperatively with
// coalesced accesses (each group of 8 lanes reads 8 consecutive groups of one
// weight row; each 4 lanes one activation row's 256 code bytes) into
// registers, then stored to LDS: the operands reach the lanes that feed
// the MFMAs from LDS, never as 32 scattered rows per load instruction.
struct ChunkRegs {
  Raw wr[2];      // weight groups: column t / 8 (+ 32), group t % 8
  v4u32 xc[4];    // activation codes: row t / 4, groups 2 (t % 4) and 2 (t % 4) + 1
  float dx[2];    // and their scales
  v4u32 xp[4];    // F8: the second half of the groups' 64-byte e4m3 planes
};



template <int F>
__device__ __forceinline__ void chunk_load(const GemmArgs& a, const uint8_t* wb, const Regions& rg,
                                           int col0, const int* sxr, int64_t xstride, int G, int gc,
                                           ChunkRegs& cr)
{
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int64_t o = min(col0 + (t >> 3) + 32 * p, a.out - 1);
    load_group<F>(wb, rg, o, G, min(gc + (t & 7), G - 1), a.in, cr.wr[p]);
  }
  const uint8_t* xr = a.xq + (int64_t)sxr[t >> 2] * xstride;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int g = min(gc + 2 * (t & 3) + k, G - 1);
    const v4u32* q = (const v4u32*)(xr + (int64_t)g * 32);
    cr.xc[2 * k] = q[0];
    cr.xc[2 * k + 1] = q[1];
    cr.dx[k] = ((const float*)(xr + a.in))[g];
  }
}

constexpr int GSW = GKC * raw_dwords<DT_Q8_0>() + 1;  // LDS dwords per weight column (odd)
constexpr int GSA = GKC * 8 + 2;                     // LDS dwords per activation row

template <int F>
__device__ __forceinline__ void chunk_store(const ChunkRegs& cr, uint32_t* sw, uint32_t* sa, double* sdx,
                                            int* sbs)
{
  const int t = threadIdx.x;
  constexpr int WS = GKC * raw_dwords<F>() + 1;  // this format's column stride
#pragma unroll
  for (int p = 0; p < 2; p++) raw_put<F>(sw + ((t >> 3) + 32 * p) * WS + (t & 7), GKC, cr.wr[p]);
  const int row = t >> 2;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int j = 2 * (t & 3) + k;
    uint32_t* d = sa + row * GSA + j * 8;
    *(v4u32*)d = cr.xc[2 * k];
    *(v4u32*)(d + 4) = cr.xc[2 * k + 1];
    sdx[j * GBM + row] = (double)cr.dx[k];  // widened once here, not per output
    if constexpr (needs_xsum(F) && F != DT_Q4_K) {  // (Q4_K: the m_j sums on the matrix cores)
      const v4u32 u0 = cr.xc[2 * k], u1 = cr.xc[2 * k + 1];
      int sm = 0;
      sm = sdot4((int)u0.x, 0x01010101, sm); sm = sdot4((int)u0.y, 0x01010101, sm);
      sm = sdot4((int)u0.z, 0x01010101, sm); sm = sdot4((int)u0.w, 0x01010101, sm);
      sm = sdot4((int)u1.x, 0x01010101, sm); sm = sdot4((int)u1.y, 0x01010101, sm);
      sm = sdot4((int)u1.z, 0x01010101, sm); sm = sdot4((int)u1.w, 0x01010101, sm);
      sbs[j * GBM + row] = sm;
    }
  }
}

// ------------------------------------------- MXFP4 on the scaled f8f6f4 MFMA
// v_mfma_scale_f32_32x32x64_f8f6f4 with B the group's e2m1 codes as they are
// stored (no decode) and A the activation codes split q = 16 hi + lo (hi, lo
// in [-8, 8]): A's first 32 k are e4m3(16 hi) and its last 32 e4m3(lo), B's
// two 32-k blocks both the group's 32 codes, every block scale 1. Each
// product is exact (e4m3 x e2m1) and every partial sum a multiple of 1/2
// below 2^23, so the f32 result is the exact group dot sum q w over the e2m1
// values, half the doubled-table integer sum of the int8 path: the CPU's
// group sum, as exact. One instruction per 32-value group, like the int8
// MFMA, without the e2m1 -> int8 decode of the weights.
//
// Operand layout (probed on gfx950): byte j of an 8-bit operand in lane half
// h holds k = 16 h + j (j < 16) or 32 + 16 h + (j - 16); nibble j of a 4-bit
// operand in lane half h holds k = 32 h + j. The k order is free as long as A
// and B agree: B's block position p is nibble p of the 16 stored code bytes,
// value v(p) = p / 2 + 16 (p % 2) (byte j: value j low, value j + 16 high), so
// A's positions take q[v(p)]. A row's planes per group (f8_planes): for h =
// 0, 1 the 32 bytes e4m3(16 hi[v(16h + j)]) j < 16, e4m3(lo[v(16h + j)]) j
// < 16 - lane half h reads bytes 32h..32h+31 of the group.
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

// e4m3 of an integer in [-8, 8] (times 16 when x16: the exponent + 4)
__device__ __forceinline__ uint32_t e4m3_small(int v, bool x16)
{
  const int a = v < 0 ? -v : v;
  // 0, 1 .. 8: 0x00 0x38 0x40 0x44 0x48 0x4A 0x4C 0x4E 0x50
  const uint32_t lo4 = 0x44403800u, hi4 = 0x4E4C4A48u;
  uint32_t m = a == 8 ? 0x50u : (a < 4 ? (lo4 >> (8 * a)) & 255u : (hi4 >> (8 * (a - 4))) & 255u);
  if (x16 && a) m += 0x20u;
  return v < 0 ? (m | 0x80u) : m;
}

template <int F>
__device__ __forceinline__ void chunk_load8(const GemmArgs& a, const uint8_t* wb, const Regions& rg,
                                            int col0, const int* sxr, int64_t xstride, int G, int gc,
                                            ChunkRegs& cr)
{
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int64_t o = min(col0 + (t >> 3) + 32 * p, a.out - 1);
    load_group<F>(wb, rg, o, G, min(gc + (t & 7), G - 1), a.in, cr.wr[p]);
  }
  const uint8_t* xr = a.xq + (int64_t)sxr[t >> 2] * xstride;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int g = min(gc + 2 * (t & 3) + k, G - 1);
    const v4u32* q = (const v4u32*)(xr + (int64_t)g * 64);
    cr.xc[2 * k] = q[0];
    cr.xc[2 * k + 1] = q[1];
    cr.xp[2 * k] = q[2];
    cr.xp[2 * k + 1] = q[3];
    cr.dx[k] = ((const float*)(xr + (int64_t)G * 64))[g];
  }
}

constexpr int GSA8 = GKC * 16 + 4;  // LDS dwords per activation row of planes

template <int F>
__device__ __forceinline__ void chunk_store8(const ChunkRegs& cr, uint32_t* sw, uint32_t* sa, double* sdx)
{
  const int t = threadIdx.x;
  constexpr int WS = GKC * raw_dwords<F>() + 1;
#pragma unroll
  for (int p = 0; p < 2; p++) raw_put<F>(sw + ((t >> 3) + 32 * p) * WS + (t & 7), GKC, cr.wr[p]);
  const int row = t >> 2;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int j = 2 * (t & 3) + k;
    uint32_t* d = sa + row * GSA8 + j * 16;
    *(v4u32*)d = cr.xc[2 * k];
    *(v4u32*)(d + 4) = cr.xc[2 * k + 1];
    *(v4u32*)(d + 8) = cr.xp[2 * k];
    *(v4u32*)(d + 12) = cr.xp[2 * k + 1];
    sdx[j * GBM + row] = (double)cr.dx[k];
  }
}

// the MXFP4 GEMM on the f8f6f4 matrix cores: gemm's tiles, chunks and
// double scaling; A from the planes of f8_planes
__device__ __forceinline__ void gemm_mxfp4_f8(const GemmArgs& a)
{
  constexpr int F = DT_MXFP4;
  __shared__ uint32_t sw_[GBN * GSW];
  __shared__ __align__(16) uint32_t sa_[GBM * GSA8];
  __shared__ __align__(16) double sdx_[GKC * GBM];
  __shared__ int sxr[GBM], syr[GBM];
  const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5;
  const int wm = w & 1, wn = w >> 1;
  const int G = a.in >> 5;
  const int64_t xstride = 68 * (int64_t)G;
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
  const int col0 = blockIdx.x * GBN;
  const int o_real = col0 + 32 * wn + (l & 31);
  const int64_t o = min(o_real, a.out - 1);
  const int rb = 32 * wm + 4 * h;
  constexpr int WS = GKC * raw_dwords<F>() + 1;
  const uint32_t* myw = sw_ + (32 * wn + (l & 31)) * WS;
  const uint32_t* mya = sa_ + (32 * wm + (l & 31)) * GSA8 + 8 * h;
  double acc[16];
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.0;
  const int nch = (G + GKC - 1) / GKC;
  ChunkRegs cr;
  chunk_load8<F>(a, wb, rg, col0, sxr, xstride, G, 0, cr);
  chunk_store8<F>(cr, sw_, sa_, sdx_);
  chunk_load8<F>(a, wb, rg, col0, sxr, xstride, G, GKC, cr);
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    const int gc = c * GKC;
#pragma unroll
    for (int j = 0; j < GKC; j++) {
      const int g = gc + j;
      if (g < G) {
        const Raw r = raw_get<F>(myw + j, GKC);
        const v4u32 a0 = *(const v4u32*)(mya + j * 16), a1 = *(const v4u32*)(mya + j * 16 + 4);
        const v8i_t av = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        const v8i_t bv = {(int)r.q0.x, (int)r.q0.y, (int)r.q0.z, (int)r.q0.w, 0, 0, 0, 0};
        const v16f_t z = {};
        // formats: A e4m3 (0), B e2m1 (4); every block scale E8M0 127 (1.0)
        const v16f_t cf = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, z, 0, 4, 0, 0x7F7F7F7F, 0,
                                                                           0x7F7F7F7F);
        const double dw = mxfp4_q8_scale(r.a);
        double2 dq[8];
#pragma unroll
        for (int q = 0; q < 8; q++) dq[q] = *(const double2*)&sdx_[j * GBM + rb + 8 * (q >> 1) + 2 * (q & 1)];
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const double2 d2 = dq[i >> 1];
          const double dx = (i & 1) ? d2.y : d2.x;
          // 2 cf: the doubled-table integer group sum of the CPU, exact
          acc[i] = __builtin_fma(2.0 * (double)cf[i], dw * dx, acc[i]);
        }
      }
    }
    __syncthreads();
    chunk_store8<F>(cr, sw_, sa_, sdx_);
    chunk_load8<F>(a, wb, rg, col0, sxr, xstride, G, gc + 2 * GKC, cr);
    __syncthreads();
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

// the e4m3 planes of quantized activation rows for gemm_mxfp4_f8: row r of
// xq (codes [in], then dx [G]) into row r of planes (64 bytes per group as
// above, then the same dx [G]); one thread per group
struct PlanesArgs {
  const uint8_t* xq;
  uint8_t* planes;
  int32_t rows, in;
};
__device__ __forceinline__ void f8_planes(const PlanesArgs& a)
{
  const int G = a.in >> 5;
  const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int row = blockIdx.y;
  if (gi >= G) return;
  const uint8_t* src = a.xq + (int64_t)row * ((int64_t)a.in + 4 * G);
  uint8_t* dst = a.planes + (int64_t)row * 68 * G;
  const v4u32 c0 = *(const v4u32*)(src + gi * 32), c1 = *(const v4u32*)(src + gi * 32 + 16);
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  uint32_t outw[16];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      uint32_t whi = 0, wlo = 0;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const int p = 16 * hh + 4 * jj + b;
        const int v = (p >> 1) + 16 * (p & 1);
        const int q = (int)(int8_t)((cw[v >> 2] >> (8 * (v & 3))) & 255u);
        const int hi = (q + 8) >> 4, lo = q - 16 * hi;
        whi |= e4m3_small(hi, true) << (8 * b);
        wlo |= e4m3_small(lo, false) << (8 * b);
      }
      outw[8 * hh + jj] = whi;
      outw[8 * hh + 4 + jj] = wlo;
    }
  v4u32* d = (v4u32*)(dst + gi * 64);
#pragma unroll
  for (int k = 0; k < 4; k++) d[k] = v4u32{outw[4 * k], outw[4 * k + 1], outw[4 * k + 2], outw[4 * k + 3]};
  ((float*)(dst + (int64_t)G * 64))[gi] = ((const float*)(src + a.in))[gi];
}

template <int F>
__device__ __forceinline__ void gemm(const GemmArgs& a)
{
  // one chunk's operands: weight groups by column, activation codes by row,
  // the rows' scales and code sums
  __shared__ uint32_t sw_[GBN * GSW];
  __shared__ __align__(16) uint32_t sa_[GBM * GSA];
  __shared__ __align__(16) double sdx_[GKC * GBM];
  __shared__ int sbs_[needs_xsum(F) ? GKC * GBM : 1];
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
  const int col0 = blockIdx.x * GBN;
  const int o_real = col0 + 32 * wn + (l & 31);
  const int64_t o = min(o_real, a.out - 1);
  const int rb = 32 * wm + 4 * h;  // tile row of result register i: rb + 8 (i / 4) + i % 4
  constexpr int WS = GKC * raw_dwords<F>() + 1;
  const uint32_t* myw = sw_ + (32 * wn + (l & 31)) * WS;     // this lane's weight column
  const uint32_t* mya = sa_ + (32 * wm + (l & 31)) * GSA;    // this lane's activation row

  double acc[16];
  int isum[16], msum[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    acc[i] = 0.0;
    isum[i] = msum[i] = 0;
  }
  // Q4_K: the super-block's minimum sum sum_j m_j bsum_j kept on the matrix
  // cores: A times the group's m_j broadcast (m < 64), accumulated over the
  // 8 groups of the super-block, exact int32
  v16i cm = {};

  // chunk c + 1 is in registers (its loads issued during chunk c - 1) while
  // chunk c is computed from LDS; loads past the last group read the last
  // group (values unused)
  const int nch = (G + GKC - 1) / GKC;
  ChunkRegs cr;
  chunk_load<F>(a, wb, rg, col0, sxr, xstride, G, 0, cr);
  chunk_store<F>(cr, sw_, sa_, sdx_, sbs_);
  chunk_load<F>(a, wb, rg, col0, sxr, xstride, G, GKC, cr);
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    const int gc = c * GKC;
#pragma unroll
    for (int j = 0; j < GKC; j++) {
      const int g = gc + j;
      if (g < G) {
        const Raw r = raw_get<F>(myw + j, GKC);
        const uint2 x0 = *(const uint2*)(mya + j * 8 + 2 * h);
        const uint2 x1 = *(const uint2*)(mya + j * 8 + 4 + 2 * h);
        double (*sdx)[GBM] = (double (*)[GBM])sdx_;
        int (*sbs)[GBM] = (int (*)[GBM])sbs_;
        const int buf = 0;
        (void)buf;
          const v4i bv = b_operand<F>(r, h);
          v16i s;
          v16i s2 = {};
          if constexpr (F == DT_Q4_K) {
            int sc, mn;
            scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, mn);
            const int mb = (int)(((uint32_t)mn * 0x010101u) | ((uint32_t)mn << 24));
            const v4i bm = {mb, mb, mb, mb};
            const v4i av = {(int)x0.x, (int)x0.y, (int)x1.x, (int)x1.y};
            const v16i z = {};
            s = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, z, 0, 0, 0);
            cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bm, (g & 7) == 0 ? z : cm, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) isum[i] += __mul24(sc, s[i]);  // |sums| < 2^16, sc < 64
            if ((g & 7) == 7) {  // (Q4_K rows hold whole super-blocks)
              const double hd = half_to_float(r.q1.x & 0xffffu), hm = half_to_float(r.q1.x >> 16);
#pragma unroll
              for (int i = 0; i < 16; i++) {
                const double dx = sdx[j][rb + 8 * (i >> 2) + (i & 3)];
                acc[i] = acc[i] + ((hd * dx) * (double)isum[i] - (hm * dx) * (double)cm[i]);
                isum[i] = 0;
              }
            }
            continue;
          }
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
              // |sums| < 2^16, scales < 64: 24-bit multiplies
              isum[i] += __mul24(sc, s[i]);
              msum[i] += __mul24(mn, sbs[j][rb + 8 * (i >> 2) + (i & 3)]);
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
            for (int i = 0; i < 16; i++) isum[i] += __mul24(sa, s[i]) + __mul24(sb, s2[i]);
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
            // s * dw * dx is exact in double (at most 19 + 11 + 11 significant
            // bits), so one fused multiply-add rounds as the CPU's multiply-then-add
            // the 16 rows' scales: four 16-byte LDS reads, all issued first
            double2 dq[8];
#pragma unroll
            for (int q = 0; q < 8; q++) dq[q] = *(const double2*)&sdx[j][rb + 8 * (q >> 1) + 2 * (q & 1)];
#pragma unroll
            for (int i = 0; i < 16; i++) {
              const double2 d2 = dq[i >> 1];
              const double dx = (i & 1) ? d2.y : d2.x;
              acc[i] = __builtin_fma((double)s[i], dw * dx, acc[i]);
            }
          }
      }
    }
    __syncthreads();  // the chunk's LDS reads are done
    chunk_store<F>(cr, sw_, sa_, sdx_, sbs_);
    chunk_load<F>(a, wb, rg, col0, sxr, xstride, G, gc + 2 * GKC, cr);
    __syncthreads();
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

// ------------------------------------------------ a small batch of rows
// gemm8: the same arithmetic for at most 8 activation rows (blockIdx.y: a
// chunk of 8 rows, or a grouped-expert item of at most 8 slots), the weights
// streamed once: a block owns 128 outputs (4 waves of 32) and walks the
// output tiles of its grid share. Per 32-value group a wave runs the MFMA of
// the big GEMM with the rows in A lanes 0..7 (lanes 8..31 zero): of its
// result registers, 0..3 hold the 8 rows x 32 outputs, one (row, output) per
// lane and register, so the scaling in double wastes no lane. The chunks of
// GKC groups (128 weight columns, 8 activation rows) are loaded coalesced
// into registers a chunk ahead, then through LDS to the lanes.
constexpr int G8N = 128;  // outputs of a block tile

struct Chunk8 {
  Raw wr[4];    // weight groups: column t / 8 + 32 p, group t % 8
  v4u32 xc[2];  // activation codes (t < 64): row t / 8, group t % 8
  float dx;
};

template <int F>
__device__ __forceinline__ void chunk8_load(const GemmArgs& a, const uint8_t* wb, const Regions& rg,
                                            int col0, const int* sxr, int64_t xstride, int G, int gc,
                                            Chunk8& cr)
{
  const int t = threadIdx.x;
  const int g = min(gc + (t & 7), G - 1);
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int64_t o = min(col0 + (t >> 3) + 32 * p, a.out - 1);
    load_group<F, true>(wb, rg, o, G, g, a.in, cr.wr[p]);
  }
  if (t < 64) {
    const uint8_t* xr = a.xq + (int64_t)sxr[t >> 3] * xstride;
    const v4u32* q = (const v4u32*)(xr + (int64_t)g * 32);
    cr.xc[0] = q[0];
    cr.xc[1] = q[1];
    cr.dx = ((const float*)(xr + a.in))[g];
  }
}

template <int F>
__device__ __forceinline__ void chunk8_store(const Chunk8& cr, uint32_t* sw, uint32_t* sa, float* sdx,
                                             int* sbs)
{
  const int t = threadIdx.x;
  constexpr int WS = GKC * raw_dwords<F>() + 1;
#pragma unroll
  for (int p = 0; p < 4; p++) raw_put<F>(sw + ((t >> 3) + 32 * p) * WS + (t & 7), GKC, cr.wr[p]);
  if (t < 64) {
    const int row = t >> 3, j = t & 7;
    uint32_t* d = sa + row * GSA + j * 8;
    *(v4u32*)d = cr.xc[0];
    *(v4u32*)(d + 4) = cr.xc[1];
    sdx[j * 8 + row] = cr.dx;
    if constexpr (needs_xsum(F)) {
      const v4u32 u0 = cr.xc[0], u1 = cr.xc[1];
      int sm = 0;
      sm = sdot4((int)u0.x, 0x01010101, sm); sm = sdot4((int)u0.y, 0x01010101, sm);
      sm = sdot4((int)u0.z, 0x01010101, sm); sm = sdot4((int)u0.w, 0x01010101, sm);
      sm = sdot4((int)u1.x, 0x01010101, sm); sm = sdot4((int)u1.y, 0x01010101, sm);
      sm = sdot4((int)u1.z, 0x01010101, sm); sm = sdot4((int)u1.w, 0x01010101, sm);
      sbs[j * 8 + row] = sm;
    }
  }
}

template <int F>
__device__ __forceinline__ void gemm8(const GemmArgs& a)
{
  constexpr int WS = GKC * raw_dwords<F>() + 1;
  __shared__ uint32_t sw_[G8N * WS];
  __shared__ __align__(16) uint32_t sa_[8 * GSA];
  __shared__ __align__(16) float sdx_[GKC * 8];
  __shared__ int sbs_[needs_xsum(F) ? GKC * 8 : 1];
  __shared__ int sxr[8], syr[8];
  const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5;
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
    nrows = min(8, it.z);
    if (t < 8) {
      const int sl = a.perm[it.y + min(t, nrows - 1)];
      sxr[t] = a.x_per_slot ? sl / a.x_per_slot : 0;
      syr[t] = sl;
    }
  } else {
    const int r0 = blockIdx.y * 8;
    nrows = min(8, a.rows - r0);
    if (t < 8) sxr[t] = syr[t] = r0 + min(t, nrows - 1);
  }
  __syncthreads();
  const Regions rg = regions(F, a.out, a.in);
  const int ntiles = (a.out + G8N - 1) / G8N;
  const int nch = (G + GKC - 1) / GKC;
  // this block's (tile, chunk) steps, tile-major: step q is chunk q % nch of
  // tile blockIdx.x + (q / nch) gridDim.x
  const int mytiles = ((int)blockIdx.x < ntiles) ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int nsteps = mytiles * nch;
  if (nsteps == 0) return;
  const int arow = l & 31;  // A lane: row arow (rows 8.. are zero)
  const uint32_t* myw = sw_ + (32 * w + (l & 31)) * WS;
  const uint32_t* mya = sa_ + min(arow, 7) * GSA;
  auto step_at = [&](int q, int& col0, int& gc) {
    col0 = ((int)blockIdx.x + (q / nch) * (int)gridDim.x) * G8N;
    gc = (q % nch) * GKC;
  };
  double acc[4];
  int isum[4], msum[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    acc[i] = 0.0;
    isum[i] = msum[i] = 0;
  }
  Chunk8 cr;
  int col0, gc;
  step_at(0, col0, gc);
  chunk8_load<F>(a, wb, rg, col0, sxr, xstride, G, gc, cr);
  chunk8_store<F>(cr, sw_, sa_, sdx_, sbs_);
  if (nsteps > 1) {
    int c1, g1;
    step_at(1, c1, g1);
    chunk8_load<F>(a, wb, rg, c1, sxr, xstride, G, g1, cr);
  }
  __syncthreads();
  for (int q = 0; q < nsteps; q++) {
    step_at(q, col0, gc);
#pragma unroll
    for (int j = 0; j < GKC; j++) {
      const int g = gc + j;
      if (g < G) {
        const Raw r = raw_get<F>(myw + j, GKC);
        uint2 x0 = *(const uint2*)(mya + j * 8 + 2 * h);
        uint2 x1 = *(const uint2*)(mya + j * 8 + 4 + 2 * h);
        if (arow >= 8) x0 = x1 = make_uint2(0u, 0u);
        const float* sdx = sdx_ + j * 8;
        const int* sbs = sbs_ + (needs_xsum(F) ? j * 8 : 0);
        const v4i bv = b_operand<F>(r, h);
        v16i s;
        v16i s2 = {};
        if constexpr (F == DT_Q6_K) {
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
        // result register i < 4 of lane l: row 4 h + i, output l % 32
        if constexpr (F == DT_Q4_K) {
          int sc, mn;
          scale_min_k4(g & 7, r.q1.y, r.q1.z, r.q1.w, sc, mn);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            isum[i] += __mul24(sc, s[i]);
            msum[i] += __mul24(mn, sbs[4 * h + i]);
          }
          if ((g & 7) == 7) {
            const double hd = half_to_float(r.q1.x & 0xffffu), hm = half_to_float(r.q1.x >> 16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const double dx = sdx[4 * h + i];
              acc[i] = acc[i] + ((hd * dx) * (double)isum[i] - (hm * dx) * (double)msum[i]);
              isum[i] = msum[i] = 0;
            }
          }
        } else if constexpr (F == DT_Q6_K) {
          const int sa = (int)(int8_t)(r.a & 255u), sb = (int)(int8_t)(r.a >> 8);
#pragma unroll
          for (int i = 0; i < 4; i++) isum[i] += __mul24(sa, s[i]) + __mul24(sb, s2[i]);
          if ((g & 7) == 7) {
            const double d = half_to_float(r.d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const double dx = sdx[4 * h + i];
              acc[i] = acc[i] + (d * dx) * (double)isum[i];
              isum[i] = 0;
            }
          }
        } else if constexpr (F == DT_Q5_1) {
          const double d = half_to_float(r.a & 0xffffu), m = half_to_float(r.a >> 16);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const double dx = sdx[4 * h + i];
            const double tt = (double)s[i] * (d * dx);
            acc[i] = acc[i] + (tt + m * (dx * (double)sbs[4 * h + i]));
          }
        } else {
          double dw;
          if constexpr (F == DT_MXFP4) dw = mxfp4_q8_scale(r.a);
          else dw = half_to_float(r.a);
          const float4 d4 = *(const float4*)&sdx[4 * h];
          const double dxs[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 4; i++) acc[i] = __builtin_fma((double)s[i], dw * dxs[i], acc[i]);
        }
      }
    }
    __syncthreads();  // the chunk's LDS reads are done
    if (q + 1 < nsteps) {
      chunk8_store<F>(cr, sw_, sa_, sdx_, sbs_);
      if (q + 2 < nsteps) {
        int c2, g2;
        step_at(q + 2, c2, g2);
        chunk8_load<F>(a, wb, rg, c2, sxr, xstride, G, g2, cr);
      }
    }
    // the tile's last chunk: its outputs, then a fresh sum
    if (q % nch == nch - 1) {
      const int o = col0 + 32 * w + (l & 31);
      if (o < a.out) {
        const double b = bias ? (double)bias[o] : 0.0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int rt = 4 * h + i;
          if (rt < nrows) {
            double v = acc[i];
            if (bias) v = b + v;
            a.y[(int64_t)syr[rt] * a.out + o] = (float)v;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        acc[i] = 0.0;
        isum[i] = msum[i] = 0;
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------- float weights
// y[r, o] = bias[o] + sum_i x[r, i] w[o, i] for F32 / BF16 / F16 weights in
// the Q8 arithmetic of TInferCpuBackend.Linear's float branch
// (backend.cpu.pas:1548-1565): every product of a float activation and a
// float weight is exact in double, and the sum runs in double, here on the
// f64 matrix cores (v_mfma_f64_16x16x4_f64; only the order of the double sum
// differs from the CPU's). A block owns 64 rows x 64 outputs, each wave
// 32 x 32 as 2 x 2 tiles of 16 x 16; chunks of FKC values of x and w are
// loaded coalesced into LDS (the next chunk's loads in flight while one is
// computed).
typedef double v4d __attribute__((ext_vector_type(4)));
constexpr int FKC = 32;  // values of the sum per chunk

template <int F>
__device__ __forceinline__ float wval(const void* w, int64_t i)
{
  if constexpr (F == DT_F32) return ((const float*)w)[i];
  else if constexpr (F == DT_BF16) return bits_float((uint32_t)((const uint16_t*)w)[i] << 16);
  else return half_to_float(((const uint16_t*)w)[i]);
}

template <int F>
__device__ __forceinline__ void gemm_flt(const GemmArgs& a)
{
  __shared__ float xs[2][GBM][FKC + 1];
  __shared__ float ws[2][GBN][FKC + 1];
  __shared__ int sxr[GBM], syr[GBM];
  const int t = threadIdx.x, l = t & 63, w = t >> 6;
  const int wm = w & 1, wn = w >> 1;
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
  const int col0 = blockIdx.x * GBN;
  // a thread's share of a chunk: 8 consecutive values of row (t / 4) of x
  // and of column (t / 4) of w
  const int lr = t >> 2, lk = 8 * (t & 3);
  const float* xrow = a.x + (int64_t)sxr[lr] * a.in;
  const int64_t wrow = (int64_t)min(col0 + lr, a.out - 1) * a.in;
  // this block's values of the sum: [kb, ke)
  const int kb = a.ksplit > 1 ? (int)blockIdx.z * a.klen : 0;
  const int ke = a.ksplit > 1 ? min(a.in, kb + a.klen) : a.in;
  float xv[8], wv[8];
  auto load = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int k = min(k0 + lk + u, ke - 1);
      xv[u] = xrow[k];
      wv[u] = wval<F>(wb, wrow + k);
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      xs[buf][lr][lk + u] = xv[u];
      ws[buf][lr][lk + u] = wv[u];
    }
  };
  v4d acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
  const int nch = (ke - kb + FKC - 1) / FKC;
  load(kb);
  store(0);
  __syncthreads();
  // operand lane mapping of v_mfma_f64_16x16x4_f64 (probed on gfx950): A
  // lane l = row l % 16, k = l / 16; B lane l = column l % 16, k = l / 16;
  // result register e of lane l = row 4 e + l / 16, column l % 16
  const int ar = l & 15, ak = l >> 4;
  for (int c = 0; c < nch; c++) {
    const int buf = c & 1, k0 = kb + c * FKC;
    if (c + 1 < nch) load(k0 + FKC);
#pragma unroll
    for (int kk = 0; kk < FKC; kk += 4) {
      // a chunk past the end of the sum: values beyond in read 0 weight
      const bool kin = k0 + kk + ak < ke;
      double av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; i++) av[i] = (double)xs[buf][32 * wm + 16 * i + ar][kk + ak];
#pragma unroll
      for (int j = 0; j < 2; j++) bv[j] = kin ? (double)ws[buf][32 * wn + 16 * j + ar][kk + ak] : 0.0;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (c + 1 < nch) store(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int o = col0 + 32 * wn + 16 * j + ar;
    if (o >= a.out) continue;
    const double b = bias ? (double)bias[o] : 0.0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int rt = 32 * wm + 16 * i + 4 * e + ak;
        if (rt < nrows) {
          double v = acc[i][j][e];
          if (a.ksplit > 1) {
            a.part[((int64_t)blockIdx.z * a.rows + syr[rt]) * a.out + o] = v;
            continue;
          }
          if (bias) v = b + v;
          a.y[(int64_t)syr[rt] * a.out + o] = (float)v;
        }
      }
  }
}

}  // namespace ihip

// (three blocks a CU: the registers fit in 168, no spill; a b512 6144 x 2048
// launch's 768 blocks then run in one round instead of one and a half)
#define IHIP_GEMM(NAME, F)                                                                      \
  extern "C" __global__ __launch_bounds__(256, 3) void gemm_##NAME(ihip::GemmArgs a) { ihip::gemm<F>(a); } \
  extern "C" __global__ __launch_bounds__(256) void gemm8_##NAME(ihip::GemmArgs a)                    \
  {                                                                                                 \
    ihip::touch_kernargs<sizeof(ihip::GemmArgs)>();                                                 \
    ihip::gemm8<F>(a);                                                                              \
  }

#define IHIP_GEMM_FLT(NAME, F) \
  extern "C" __global__ __launch_bounds__(256) void gemm_##NAME(ihip::GemmArgs a) { ihip::gemm_flt<F>(a); }

#ifdef IHIP_ONLY_FMT_Q8_0
IHIP_GEMM(q8_0, ihip::DT_Q8_0)
#endif
#ifdef IHIP_ONLY_FMT_F32
IHIP_GEMM_FLT(f32, ihip::DT_F32)
#endif
#ifdef IHIP_ONLY_FMT_BF16
IHIP_GEMM_FLT(bf16, ihip::DT_BF16)
#endif
#ifdef IHIP_ONLY_FMT_F16
IHIP_GEMM_FLT(f16, ihip::DT_F16)
#endif
#ifdef IHIP_ONLY_FMT_Q4_0
IHIP_GEMM(q4_0, ihip::DT_Q4_0)
#endif
#ifdef IHIP_ONLY_FMT_MXFP4
extern "C" __global__ __launch_bounds__(256) void gemm_mxfp4_f8(ihip::GemmArgs a) { ihip::gemm_mxfp4_f8(a); }
extern "C" __global__ __launch_bounds__(256) void f8_planes(ihip::PlanesArgs a) { ihip::f8_planes(a); }
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
