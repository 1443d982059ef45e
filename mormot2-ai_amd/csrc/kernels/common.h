// common.h - device helpers shared by the gfx950 kernels of mormot.ai.infer.hip.
// Compiled with -ffp-contract=off: a float expression rounds every step, as
// the reference's Pascal does; a fused multiply-add is always written out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../layout.h"

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

__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int& sc, int& m)
{
  if (j < 4) {
    sc = (int)(byte_of(s0, s1, s2, j) & 63u);
    m = (int)(byte_of(s0, s1, s2, j + 4) & 63u);
  } else {
    uint32_t a = byte_of(s0, s1, s2, j + 4);
    sc = (int)((a & 15u) | ((byte_of(s0, s1, s2, j - 4) >> 6) << 4));
    m = (int)((a >> 4) | ((byte_of(s0, s1, s2, j) >> 6) << 4));
  }
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

template <typename T>
__device__ __forceinline__ T wave_sum(T v, int width)
{
  for (int o = 1; o < width; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

}  // namespace ihip
