// common.h - device helpers shared by the gfx950 kernels of mormot.ai.infer.hip.
// Compiled with -ffp-contract=off: a float expression rounds every step, as
// the reference's Pascal does; a fused multiply-add is always written out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../layout.h"

// IHIP_STAMP(i): with IHIP_TRACE defined (a timing build that defines
// ihip_trace), the 100 MHz clock at phase i of an instrumented kernel, held
// in registers and written by thread 0 of the block when the function that
// opened IHIP_STAMP_SCOPE returns (a store per stamp would make the
// compiler wait for the vector memory counter at the next stamp); compiled
// out otherwise
#ifdef IHIP_TRACE
// the stamp buffer of a timing build ([blocks][8] clocks), set by
// ihip_trace_buffer through hipModuleGetGlobal
__constant__ uint64_t* ihip_trace;  // scalar loads
struct IhipStamps {
  uint64_t t[8];
  uint32_t mask = 0;
  __device__ ~IhipStamps()
  {
    if (threadIdx.x == 0 && ihip_trace) {
      uint64_t* p = ihip_trace + (((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 8;
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (mask & (1u << i)) p[i] = t[i];
    }
  }
};
#define IHIP_STAMP_SCOPE IhipStamps ihip_st
#define IHIP_STAMP(i)                                   \
  do {                                                  \
    ihip_st.t[i] = __builtin_amdgcn_s_memrealtime();    \
    ihip_st.mask |= 1u << (i);                          \
  } while (0)
#else
#define IHIP_STAMP_SCOPE \
  do {                   \
  } while (0)
#define IHIP_STAMP(i) \
  do {                \
  } while (0)
#endif

namespace ihip {

__device__ __forceinline__ float half_to_float(uint32_t h)
{
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// round to nearest even, subnormal halves included (InferSingleToHalf,
// tensor.pas:328-377, is IEEE conversion spelled out)
__device__ __forceinline__ uint16_t float_to_half(float f)
{
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bits_float(uint32_t b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ uint32_t float_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// 2^(e - 128), subnormal for e < 2 (InferE8M0HalfBits, tensor.pas:459-465)
__device__ __forceinline__ float e8m0_half(uint32_t e)
{
  return bits_float(e < 2u ? (0x00200000u << e) : ((e - 1u) << 23));
}

// the FP16 scale of an E8M0 exponent inside the exact range 104..143, else 0
// (InitMxfp4Half, backend.cpu.pas:1135-1151): 2^(e - 128) is a half there
__device__ __forceinline__ double mxfp4_q8_scale(uint32_t e)
{
  return (e >= 104u && e <= 143u) ? (double)e8m0_half(e) : 0.0;
}

__device__ __forceinline__ int sdot4(int a, int b, int c)
{
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// the doubled E2M1 values of 4 nibbles (one per byte, 0..15) as 4 int8:
// INFER_MXFP4_VALUES (tensor.pas:205-206) through two byte permutes
__device__ __forceinline__ uint32_t mxfp4_bytes(uint32_t nib)
{
  uint32_t sel = nib & 0x07070707u;
  uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
  uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
  uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (neg & m) | (pos & ~m);
}

// the 4-bit (Q4_K) scale and minimum of sub-block j (InferScaleMinK4,
// tensor.pas:379-391); s = the 12 scale bytes as 3 dwords
__device__ __forceinline__ uint32_t byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int k)
{
  uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
  return (w >> ((k & 3) * 8)) & 255u;
}

// Branch-free (j may differ between the lanes of a wave): both forms use
// byte j & 3 of each of the three dwords.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int& sc, int& m)
{
  const uint32_t sh = 8u * (uint32_t)(j & 3);
  const uint32_t b0 = (s0 >> sh) & 255u, b1 = (s1 >> sh) & 255u, b2 = (s2 >> sh) & 255u;
  const uint32_t lo_sc = b0 & 63u, lo_m = b1 & 63u;
  const uint32_t hi_sc = (b2 & 15u) | ((b0 & 0xC0u) >> 2), hi_m = (b2 >> 4) | ((b1 & 0xC0u) >> 2);
  sc = (int)(j < 4 ? lo_sc : hi_sc);
  m = (int)(j < 4 ? lo_m : hi_m);
}

// TInferCpuBackend.SwiGlu (backend.cpu.pas:1797-1834) of one value pair:
// silu(g) * u, or with limit > 0 the clamped gpt-oss form; every step
// rounded to single, the exponential in double
__device__ __forceinline__ float swiglu_value(float g, float u, float alpha, float limit)
{
  if (limit > 0) {
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    else if (u < -limit) u = -limit;
    float b = g * alpha;
    double d = b;
    b = (float)(1.0 / (1.0 + exp(-d)));
    b = g * b;
    u = u + 1.0f;
    return u * b;
  }
  double d = g;
  float b = (float)(d / (1.0 + exp(-d)));
  return b * u;
}

// TInferCpuBackend.GeluTanhGlu (backend.cpu.pas:1836-1860) of one value
// pair: gelu_tanh(g) in double (tanh as 1 - 2 / (exp(2t) + 1), +-1 beyond
// 20) rounded to single, then the product
__device__ __forceinline__ float geglu_value(float gf, float u)
{
  const double g = gf;
  double t = 0.7978845608028654 * (g + 0.044715 * g * g * g);
  if (t > 20) t = 1;
  else if (t < -20) t = -1;
  else t = 1 - 2 / (exp(2 * t) + 1);
  const float b = (float)(0.5 * g * (1 + t));
  return b * u;
}

// the fused gate/up activation: GeGLU when limit < 0, else SwiGLU
__device__ __forceinline__ float glu_value(float g, float u, float alpha, float limit)
{
  return limit < 0 ? geglu_value(g, u) : swiglu_value(g, u, alpha, limit);
}

// ------------------------------------------- results handed between blocks
// A block that hands results to the launch's last block (which counts the
// others in with an atomic counter) writes them with agent-scope stores and
// the last block reads them with agent-scope loads: both go through to the
// device's coherence point, so the blocks of different XCDs (each with its
// own L2) meet without an L2 write-back and invalidation per block (the
// cost of a device-scope fence). wait_stores() completes a block's stores
// before it counts itself.
__device__ __forceinline__ void store_agent(float* p, float v)
{
  __hip_atomic_store((uint32_t*)p, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(double* p, double v)
{
  __hip_atomic_store((uint64_t*)p, __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p)
{
  return __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ double load_agent(const double* p)
{
  return __builtin_bit_cast(double, __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}
// the kernel's argument block (BYTES of explicit arguments, then the hidden
// ones with the grid size) read into the scalar cache in one round trip at
// entry: the compiler loads each field where it is first used, and a field
// in a line not yet cached then costs a memory round trip of its own, one
// after another, before the first weight load is issued
template <int BYTES>
__device__ __forceinline__ void touch_kernargs()
{
  const uint32_t* kp = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t acc = 0;
#pragma unroll
  for (int o = 0; o < BYTES + 64; o += 64) acc ^= kp[o / 4];
  __asm__ volatile("; kernargs %0" ::"s"(acc));
}
__device__ __forceinline__ void wait_stores() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// the launch's last block to arrive (all of the block's stores complete
// first); every thread calls it, every thread gets the answer. XCD: the
// blocks that count on this counter all run on one XCD (their launch-order
// ids are equal modulo 8, and workgroups are dispatched to the 8 XCDs in
// turn), so the XCD's L2 is their point of coherence: their plain stores and
// an atomic executed in that L2 suffice, with no round trip to memory;
// otherwise the stores and the count are agent-scope (memory).
__device__ __forceinline__ bool last_block(int* counter, int blocks, bool xcd = false)
{
  __shared__ int last;
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    last = (xcd ? __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                : __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) ==
           blocks - 1;
  __syncthreads();
  return last;
}
// a load of another block's store on the same XCD (through the L2, after
// last_block with xcd)
__device__ __forceinline__ double load_xcd(const double* p)
{
  return __builtin_bit_cast(double, __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_WORKGROUP));
}

// ------------------------------------------------ wave reductions in VGPRs
// xpart<K>(v): the value of a lane in the sibling block of K lanes (the block
// that differs in lane bit K), moved inside the register file: DPP quad
// permutes (K 1, 2), row half-mirror and mirror (K 4, 8), and gfx950's
// permlane16/32 swaps (K 16, 32). For K 4 and 8 the partner is the mirrored
// lane, not lane ^ K: use it in a butterfly that starts at K = 1, where every
// lane of a block holds the same value by then. K 1, 2, 16 and 32 are lane ^ K.
template <int K>
__device__ __forceinline__ uint32_t xpart_u(uint32_t v)
{
  // every lane reads a lane of its own row: no old value is needed
  if constexpr (K == 1) return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (K == 2) return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (K == 4) return __builtin_amdgcn_update_dpp(0u, v, 0x141, 0xF, 0xF, false);
  else if constexpr (K == 8) return __builtin_amdgcn_update_dpp(0u, v, 0x140, 0xF, 0xF, false);
  else if constexpr (K == 16) {
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? p[0] : p[1];
  } else {
    static_assert(K == 32, "xpart: K is 1, 2, 4, 8, 16 or 32");
    auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? p[0] : p[1];
  }
}

template <int K, typename T>
__device__ __forceinline__ T xpart(T v)
{
  if constexpr (sizeof(T) == 8) {
    uint64_t b = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = xpart_u<K>((uint32_t)b), hi = xpart_u<K>((uint32_t)(b >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, xpart_u<K>(__builtin_bit_cast(uint32_t, v)));
  }
}

// xswap<K>(v): the value of lane ^ K for every K (K 4 and 8 as two
// bank-masked row shifts: banks that read upward, then banks that read
// downward), for reductions whose lanes of a block hold different values
template <int K>
__device__ __forceinline__ uint32_t xswap_u(uint32_t v)
{
  if constexpr (K == 4) {
    const uint32_t t = __builtin_amdgcn_update_dpp(0u, v, 0x104, 0xF, 0x5, false);
    return __builtin_amdgcn_update_dpp(t, v, 0x114, 0xF, 0xA, false);
  } else if constexpr (K == 8) {
    const uint32_t t = __builtin_amdgcn_update_dpp(0u, v, 0x108, 0xF, 0x3, false);
    return __builtin_amdgcn_update_dpp(t, v, 0x118, 0xF, 0xC, false);
  } else {
    return xpart_u<K>(v);
  }
}

template <int K, typename T>
__device__ __forceinline__ T xswap(T v)
{
  if constexpr (sizeof(T) == 8) {
    uint64_t b = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = xswap_u<K>((uint32_t)b), hi = xswap_u<K>((uint32_t)(b >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, xswap_u<K>(__builtin_bit_cast(uint32_t, v)));
  }
}

// the sums of 8 values (one per row) over aligned blocks of `width` lanes,
// transposed: at each of the levels 1, 2 and 4 a lane keeps half of its
// values and adds its partner's half, so after them it holds one row, row
// 4*bit0 + 2*bit1 + bit2 of its lane (with fewer levels, rows base + i for
// i < 8 >> levels); the tree per row is wave_sum's, level by level, own +
// partner, so every row's sum has wave_sum's bits. Returns the count of
// values left (8, 4, 2 or 1), in v[0..count).
template <typename T>
__device__ __forceinline__ int rows_sum8(T (&v)[8], int width, int& base)
{
  const int lane = threadIdx.x;
  int n = 8;
  base = 0;
  if (width > 1) {
    const bool b = lane & 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const T s = b ? v[i] : v[i + 4], k = b ? v[i + 4] : v[i];
      v[i] = k + xswap<1>(s);
    }
    n = 4;
    base += b ? 4 : 0;
  }
  if (width > 2) {
    const bool b = lane & 2;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const T s = b ? v[i] : v[i + 2], k = b ? v[i + 2] : v[i];
      v[i] = k + xswap<2>(s);
    }
    n = 2;
    base += b ? 2 : 0;
  }
  if (width > 4) {
    const bool b = lane & 4;
    const T s = b ? v[0] : v[1], k = b ? v[1] : v[0];
    v[0] = k + xswap<4>(s);
    n = 1;
    base += b ? 1 : 0;
  }
  if (width > 8) v[0] = v[0] + xswap<8>(v[0]);
  if (width > 16) v[0] = v[0] + xswap<16>(v[0]);
  if (width > 32) v[0] = v[0] + xswap<32>(v[0]);
  return n;
}

// the sum over aligned blocks of `width` lanes (1..64, a power of two), in
// every lane of the block: own + partner at each level, so the result is the
// one of the lane ^ K butterfly bit for bit
template <typename T>
__device__ __forceinline__ T wave_sum(T v, int width)
{
  if (width > 1) v = v + xpart<1>(v);
  if (width > 2) v = v + xpart<2>(v);
  if (width > 4) v = v + xpart<4>(v);
  if (width > 8) v = v + xpart<8>(v);
  if (width > 16) v = v + xpart<16>(v);
  if (width > 32) v = v + xpart<32>(v);
  return v;
}

// one butterfly level of "the first value of the largest magnitude": the
// larger magnitude, the lower index on a tie (InferQuantizeRowQ8_K's scan)
template <int K>
__device__ __forceinline__ void first_max(float& amax, float& m, int& idx)
{
  const float oa = xpart<K>(amax), om = xpart<K>(m);
  const int oi = xpart<K>(idx);
  if (oa > amax || (oa == amax && oi < idx)) {
    amax = oa;
    m = om;
    idx = oi;
  }
}

// the maximum over the wave, in every lane
template <typename T>
__device__ __forceinline__ T wave_max(T v)
{
  T o;
  o = xpart<1>(v); if (o > v) v = o;
  o = xpart<2>(v); if (o > v) v = o;
  o = xpart<4>(v); if (o > v) v = o;
  o = xpart<8>(v); if (o > v) v = o;
  o = xpart<16>(v); if (o > v) v = o;
  o = xpart<32>(v); if (o > v) v = o;
  return v;
}

}  // namespace ihip
