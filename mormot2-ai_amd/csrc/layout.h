// layout.h - the HIP device layout of a weight matrix (host and device code).
//
// A GGUF block row interleaves scales and codes in blocks of 17..210 bytes,
// most of them only 1- or 2-byte aligned: a poor fit for the 16-byte vector
// loads of a gfx950 wave. The backend owns its device copy
// (src/infer/mormot.ai.infer.backend.cuda.pas:414-449 keeps one per host
// tensor), so every matrix is repacked at upload into regions of equal-sized
// elements: all codes first, then all scales. The byte size of a matrix is
// unchanged, so matrix m of a [count, out, in] tensor still starts at
// m * out * rowbytes, as on the host (the expert stride of
// EnqueueLinearIds, backend.cuda.pas:386-412, keeps its meaning).
//
// The unit of work is a group of 32 consecutive values of a row (G = in / 32
// groups per row). Every 4-bit format stores a group as 16 bytes: byte j holds
// value j in its low and value j + 16 in its high nibble (the Q4_0 order);
// Q4_K and Q6_K are reordered into it from their GGUF super-block order.
//
//   Q8_0 : Q int8 [out][2][G][16] (per row: the first 16 values of every
//          group, then their last 16)  | S fp16 [out][G]
//   Q4_0 : Q u8 [out][G][16]              | S fp16 [out][G]
//   MXFP4: Q u8 [out][G][16]              | S e8m0 u8 [out][G]
//   Q5_0 : Q u8 [out][G][16] | H u32 [out][G] (bit v: 5th bit of value v)
//                                         | S fp16 [out][G]
//   Q5_1 : Q u8 [out][G][16] | H u32 [out][G] | S u32 [out][G] (d | m << 16)
//   Q4_K : Q u8 [out][G][16]              | S [out][NB][16] (d, dmin, the 12
//          scale bytes, as in the GGUF super-block header)
//   Q6_K : Q u8 [out][G][16] (low 4 bits) | H [out][G][8] (high 2 bits: dword
//          A for values 0..15, B for 16..31; byte i bits 2d..2d+1 hold value
//          4d + i of its half) | SC int8 [out][NB][16] | D fp16 [out][NB]
//   F32, F16, BF16: unchanged [out][in]
#pragma once

#include <stdint.h>

namespace ihip {

// TInferDType ordinals (tensor.pas:47-62)
enum : int {
  DT_F32 = 1, DT_F16 = 2, DT_BF16 = 3, DT_Q8_0 = 8, DT_Q4_0 = 9, DT_Q4_K = 10,
  DT_Q6_K = 11, DT_Q5_0 = 12, DT_MXFP4 = 13, DT_Q5_1 = 14
};

#if defined(__HIPCC__)
#define IHIP_HD __host__ __device__ inline
#else
#define IHIP_HD inline
#endif

// values per block and bytes per block (tensor.pas:187-192)
IHIP_HD int block_values(int t)
{
  switch (t) {
  case DT_F32: case DT_F16: case DT_BF16: return 1;
  case DT_Q4_K: case DT_Q6_K: return 256;
  case DT_Q8_0: case DT_Q4_0: case DT_Q5_0: case DT_MXFP4: case DT_Q5_1: return 32;
  default: return 0;
  }
}

IHIP_HD int block_bytes(int t)
{
  switch (t) {
  case DT_F32: return 4;
  case DT_F16: case DT_BF16: return 2;
  case DT_Q8_0: return 34;
  case DT_Q4_0: return 18;
  case DT_Q4_K: return 144;
  case DT_Q6_K: return 210;
  case DT_Q5_0: return 22;
  case DT_MXFP4: return 17;
  case DT_Q5_1: return 24;
  default: return 0;
  }
}

IHIP_HD uint64_t row_bytes(int t, int64_t in)
{
  return (uint64_t)(in / block_values(t)) * (uint64_t)block_bytes(t);
}

// byte offsets of the regions of one [out, in] matrix from its base
struct Regions {
  uint64_t q, h, s, s2;
};

IHIP_HD Regions regions(int t, int64_t out, int64_t in)
{
  Regions r = {0, 0, 0, 0};
  uint64_t G = (uint64_t)(in / 32), O = (uint64_t)out, NB = (uint64_t)(in / 256);
  switch (t) {
  case DT_Q8_0: r.s = O * (uint64_t)in; break;
  case DT_Q4_0: case DT_MXFP4: case DT_Q4_K: r.s = O * G * 16; break;
  case DT_Q5_0: case DT_Q5_1: r.h = O * G * 16; r.s = r.h + O * G * 4; break;
  case DT_Q6_K: r.h = O * G * 16; r.s = r.h + O * G * 8; r.s2 = r.s + O * NB * 16; break;
  default: break;
  }
  return r;
}

}  // namespace ihip
