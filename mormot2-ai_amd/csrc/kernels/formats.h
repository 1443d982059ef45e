// formats.h - the HIP weight layout of layout.h read by the gfx950 kernels:
// one 32-value group of a row as raw registers, and its code bytes.
#pragma once

#include "common.h"

namespace ihip {

// A group of 32 values as raw registers.

struct Raw {
  uint4 q0, q1;  // codes: 16 or 32 bytes
  uint32_t a, b, c, d;  // scales, high bits, header words
};

// the loads of group g of row o. Offsets are 32-bit (a matrix is below
// 4 GiB): a uniform base plus a 32-bit per-lane offset, the addressing form of
// the vector memory instructions, with no 64-bit arithmetic per lane
template <typename T>
__device__ __forceinline__ T at(const uint8_t* base, uint32_t byte_off)
{
  return *(const T*)(base + byte_off);
}

// a streamed load (NT: non-temporal, the weights of a GEMV read once per
// pass; the GEMM, which re-reads them per row tile, keeps them cached)
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));
template <typename T, bool NT>
__device__ __forceinline__ T ld(const uint8_t* base, uint32_t byte_off)
{
  if constexpr (!NT) {
    return *(const T*)(base + byte_off);
  } else if constexpr (sizeof(T) == 16) {
    const v4u32 v = __builtin_nontemporal_load((const v4u32*)(base + byte_off));
    return __builtin_bit_cast(T, v);
  } else if constexpr (sizeof(T) == 8) {
    const v2u32 v = __builtin_nontemporal_load((const v2u32*)(base + byte_off));
    return __builtin_bit_cast(T, v);
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_nontemporal_load((const uint32_t*)(base + byte_off)));
  } else if constexpr (sizeof(T) == 2) {
    return __builtin_bit_cast(T, __builtin_nontemporal_load((const uint16_t*)(base + byte_off)));
  } else {
    return __builtin_bit_cast(T, __builtin_nontemporal_load((const uint8_t*)(base + byte_off)));
  }
}

// QH (Q4_K): each lane of an aligned quad loads one dword of the 16-byte
// super-block header (lane & 3), and expand_header() hands every lane all four
// after the load; the quad's lanes must read one super-block (lanes per row a
// multiple of 8, whole quads active)
template <int F, bool NT = false, bool QH = false>
__device__ __forceinline__ void load_group(const uint8_t* w, const Regions& rg, int64_t o,
                                           int G, int g, int64_t in, Raw& r)
{
  const uint32_t og = (uint32_t)o * (uint32_t)G + (uint32_t)g;
  if constexpr (F == DT_Q8_0) {
    // a row's low halves of its groups, then their high halves: the lanes
    // of a row read one contiguous run per load
    const uint32_t q = (uint32_t)o * (uint32_t)in + (uint32_t)g * 16u;
    r.q0 = ld<uint4, NT>(w, q);
    r.q1 = ld<uint4, NT>(w, q + (uint32_t)(in >> 1));
    r.a = ld<uint16_t, NT>(w + rg.s, og * 2u);
  } else if constexpr (F == DT_Q4_0) {
    r.q0 = ld<uint4, NT>(w, og * 16u);
    r.a = ld<uint16_t, NT>(w + rg.s, og * 2u);
  } else if constexpr (F == DT_MXFP4) {
    r.q0 = ld<uint4, NT>(w, og * 16u);
    r.a = ld<uint8_t, NT>(w + rg.s, og);
  } else if constexpr (F == DT_Q5_0) {
    r.q0 = ld<uint4, NT>(w, og * 16u);
    r.b = ld<uint32_t, NT>(w + rg.h, og * 4u);
    r.a = ld<uint16_t, NT>(w + rg.s, og * 2u);
  } else if constexpr (F == DT_Q5_1) {
    r.q0 = ld<uint4, NT>(w, og * 16u);
    r.b = ld<uint32_t, NT>(w + rg.h, og * 4u);
    r.a = ld<uint32_t, NT>(w + rg.s, og * 4u);
  } else if constexpr (F == DT_Q4_K) {
    r.q0 = ld<uint4, NT>(w, og * 16u);
    const uint32_t hb = ((uint32_t)o * (uint32_t)(G >> 3) + (uint32_t)(g >> 3)) * 16u;
    if constexpr (QH)
      r.q1.x = ld<uint32_t, NT>(w + rg.s, hb + 4u * (threadIdx.x & 3u));
    else
      r.q1 = ld<uint4, NT>(w + rg.s, hb);
  } else if constexpr (F == DT_Q6_K) {
    const uint32_t ob = (uint32_t)o * (uint32_t)(G >> 3) + (uint32_t)(g >> 3);
    r.q0 = ld<uint4, NT>(w, og * 16u);
    const uint2 h = ld<uint2, NT>(w + rg.h, og * 8u);
    r.b = h.x;
    r.c = h.y;
    r.a = ld<uint16_t, NT>(w + rg.s, (ob * 8u + (uint32_t)(g & 7)) * 2u);
    r.d = ld<uint16_t, NT>(w + rg.s2, ob * 2u);
  }
}

// the header dwords of a QH load: dword i from lane i of the quad (DPP quad
// broadcasts)
__device__ __forceinline__ void expand_header(Raw& r)
{
  const uint32_t v = r.q1.x;
  r.q1.x = __builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, false);
  r.q1.y = __builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, false);
  r.q1.z = __builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, false);
  r.q1.w = __builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, false);
}

// float weights: 32 values of row o, group g (F32 128 bytes, BF16/F16 64)
template <int F>
__device__ __forceinline__ void load_fgroup(const uint8_t* w, int64_t o, int g, int64_t in,
                                            float (&v)[32])
{
  if constexpr (F == DT_F32) {
    const float4* p = (const float4*)(w + (o * in + (int64_t)g * 32) * 4);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 t = p[k];
      v[4 * k] = t.x;
      v[4 * k + 1] = t.y;
      v[4 * k + 2] = t.z;
      v[4 * k + 3] = t.w;
    }
  } else {
    const uint4* p = (const uint4*)(w + (o * in + (int64_t)g * 32) * 2);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      uint4 t = p[k];
      uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (F == DT_BF16) {
          v[8 * k + 2 * j] = bits_float(u[j] << 16);
          v[8 * k + 2 * j + 1] = bits_float(u[j] & 0xffff0000u);
        } else {
          v[8 * k + 2 * j] = half_to_float(u[j] & 0xffffu);
          v[8 * k + 2 * j + 1] = half_to_float(u[j] >> 16);
        }
      }
    }
  }
}

__device__ __forceinline__ uint32_t comp(const uint4& v, int d)
{
  return d == 0 ? v.x : (d == 1 ? v.y : (d == 2 ? v.z : v.w));
}

// the fifth bits of 4 values (bits 0..3 of b) moved to bit 4 of each byte
__device__ __forceinline__ uint32_t spread5(uint32_t b)
{
  return ((b & 1u) << 4) | ((b & 2u) << 11) | ((b & 4u) << 18) | ((b & 8u) << 25);
}

// the 4 code bytes of dword d of the low (hi = 0: values 4d..4d+3) or high
// (hi = 1: values 16 + 4d..) half of a group, as unsigned/signed int8
template <int F>
__device__ __forceinline__ uint32_t code_bytes(const Raw& r, int d, int hi)
{
  if constexpr (F == DT_Q8_0) {
    return comp(hi ? r.q1 : r.q0, d);
  } else {
    uint32_t q = comp(r.q0, d);
    uint32_t nib = hi ? ((q >> 4) & 0x0F0F0F0Fu) : (q & 0x0F0F0F0Fu);
    if constexpr (F == DT_MXFP4)
      return mxfp4_bytes(nib);
    else if constexpr (F == DT_Q5_0 || F == DT_Q5_1)
      return nib | spread5((r.b >> (hi * 16 + 4 * d)) & 15u);
    else if constexpr (F == DT_Q6_K)
      return nib | ((((hi ? r.c : r.b) >> (2 * d)) & 0x03030303u) << 4);
    else
      return nib;
  }
}

}  // namespace ihip
