// route.h - TDecoderModel.Route (decoder.pas:2901-2949) = route of
// ops.cu:664-720 as a block routine of 256 threads: softmax in double, the k
// highest logits (the lower id on a tie), weights rounded to single, renormed
// in pick order, then sorted by id. The pick order is a rank: logit i is the
// j-th pick when j logits are higher, or equal with a lower id; each thread
// counts it for its own logits against the row in LDS, eight 16-byte reads
// in flight. Used by the route kernel (prompt rows); a decode token is
// routed inside its expert launches by route_wave.
#pragma once

#include "common.h"

namespace ihip {

// the pick order of logit i (value v) among the E32 (padded) logits in LDS:
// the logits above it, and those equal to it with a lower id
__device__ __forceinline__ int logit_rank(const float* lg, int E32, int i, float v)
{
  int rank = 0;
  for (int j = 0; j < E32; j += 32) {
    float4 u[8];
#pragma unroll
    for (int q = 0; q < 8; q++) u[q] = *(const float4*)&lg[j + 4 * q];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int jj = j + 4 * q;
      rank += (u[q].x > v || (u[q].x == v && jj < i)) ? 1 : 0;
      rank += (u[q].y > v || (u[q].y == v && jj + 1 < i)) ? 1 : 0;
      rank += (u[q].z > v || (u[q].z == v && jj + 2 < i)) ? 1 : 0;
      rank += (u[q].w > v || (u[q].w == v && jj + 3 < i)) ? 1 : 0;
    }
  }
  return rank;
}

// a token's route in one wave, without LDS or barriers (every lane of the
// wave calls it with its route_logits; E <= 64 * NPL, K <= min(E, 8)). Logit i sits in lane
// i % 64, register i / 64, as an order-preserving key (-0 as +0; NaN and the
// padding as 0: never picked). The k-th largest key is found by bisection on
// its 32 bits (a wave ballot and popcount per bit), the picks are the keys
// above it and the lowest ids among those equal to it; sid[s] is the s-th
// smallest picked id. With W, sw[s] is its weight as route_block forms it:
// the softmax over all E logits in double (each lane's logits summed, then
// the wave tree), the pick's probability rounded to single, renormed by the
// picked weights summed in pick order (logit descending, id ascending).
// route_logits(): a lane's logits l, l + 64, l + 128, l + 192 (E <= 256), all
// loads issued together (an index past E reads the last logit, unused), so a
// caller issues them with its other first loads and waits for memory once.
__device__ __forceinline__ void route_logits(const float* logits, int E, float (&f)[4])
{
  const int l = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < 4; r++) f[r] = logits[min(l + 64 * r, E - 1)];
}

template <int NPL, bool W>
__device__ __forceinline__ void route_wave(const float (&fin)[4], int E, int K, int norm, int (&sid)[8],
                                           float (&sw)[8])
{
  const int l = threadIdx.x & 63;
  float f[NPL];
  uint32_t key[NPL];
#pragma unroll
  for (int r = 0; r < NPL; r++) f[r] = fin[r];
#pragma unroll
  for (int r = 0; r < NPL; r++) {
    const int i = l + 64 * r;
    if (i >= E) f[r] = -INFINITY;
    const uint32_t b = __builtin_bit_cast(uint32_t, f[r]);
    int k = (int)(b ^ ((b >> 31) * 0x7fffffffu));
    if (k == -1) k = 0;
    key[r] = (i < E && (b & 0x7fffffffu) <= 0x7f800000u) ? ((uint32_t)k ^ 0x80000000u) : 0u;
  }
  // the largest L with at least K keys >= L
  uint32_t L = 0;
  for (int bit = 31; bit >= 0; bit--) {
    const uint32_t c = L | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < NPL; r++) cnt += __popcll(__ballot(key[r] >= c));
    if (cnt >= K) L = c;
  }
  // the picks: above L, then the lowest ids equal to L
  uint64_t pk[NPL];
  int need = K;
#pragma unroll
  for (int r = 0; r < NPL; r++) {
    pk[r] = __ballot(key[r] > L);
    need -= __popcll(pk[r]);
  }
#pragma unroll
  for (int r = 0; r < NPL; r++) {
    uint64_t q = __ballot(key[r] == L && key[r] != 0u);
    while (need > 0 && q) {
      const uint64_t low = q & (~q + 1);
      pk[r] |= low;
      q ^= low;
      need--;
    }
  }
  // sid: the picked ids in id order
#pragma unroll
  for (int s = 0; s < 8; s++) {
    sid[s] = -1;
    sw[s] = 0.f;
  }
  int n = 0;
#pragma unroll
  for (int r = 0; r < NPL; r++) {
    uint64_t q = pk[r];
    while (q && n < 8) {
      const int bpos = __ffsll((long long)q) - 1;
      q &= q - 1;
#pragma unroll
      for (int s = 0; s < 8; s++)
        if (s == n) sid[s] = 64 * r + bpos;
      n++;
    }
  }
  if constexpr (W) {
    float mx = f[0];
#pragma unroll
    for (int r = 1; r < NPL; r++) mx = fmaxf(mx, f[r]);
    mx = wave_max(mx);
    const double m = mx;
    double sum = 0;
#pragma unroll
    for (int r = 0; r < NPL; r++)
      if (l + 64 * r < E) sum = sum + exp((double)f[r] - m);
    sum = wave_sum(sum, 64);
    // lane s < n: pick s (in id order), its weight and its place in pick
    // order (logit descending, id ascending) against the other picks
    int myid = -1;
#pragma unroll
    for (int s = 0; s < 8; s++) myid = l == s ? sid[s] : myid;
    // the pick's logit from the lane that holds it (no memory round trip)
    float v = -INFINITY;
#pragma unroll
    for (int r = 0; r < NPL; r++) {
      const float fr = __shfl(f[r], myid & 63);
      v = (myid >= 0 && (myid >> 6) == r) ? fr : v;
    }
    float w = myid >= 0 ? (float)(exp((double)v - m) / sum) : 0.f;
    int prank = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const float vt = __shfl(v, t);
      const int it = __shfl(myid, t);
      prank += (t < n && t != l && (vt > v || (vt == v && it < myid))) ? 1 : 0;
    }
    if (norm) {
      double picked = 0;
      for (int k = 0; k < n; k++) {
        const int who = __ffsll((long long)__ballot(l < n && prank == k)) - 1;
        picked = picked + (double)__shfl(w, who);
      }
      w = (float)((double)w / picked);
    }
#pragma unroll
    for (int s = 0; s < 8; s++) sw[s] = __shfl(w, s);
  }
}

// E <= EMAX logits, K <= 64 picks; every thread of the block calls it; on
// return sid[0..K) / sw[0..K) (LDS of the caller) hold the picks sorted by id
template <int EMAX>
__device__ __forceinline__ void route_block(const float* logits, int E, int K, int norm, int* sid,
                                            float* sw)
{
  __shared__ __align__(16) float lg[EMAX + 32];  // the row's logits, padded to 32
  __shared__ float pw[64];                       // the picks' weights and ids in pick order
  __shared__ int pid[64];
  const int t = threadIdx.x, l = t & 63;
  const int E32 = (E + 31) & ~31;
  for (int i = t; i < E; i += 256) lg[i] = logits[i];
  // below every logit and never the lower id: the padding is no pick
  if (E + t < E32) lg[E + t] = -INFINITY;
  __syncthreads();
  // every wave forms the same maximum and sum
  float mx = -INFINITY;
  for (int i = l; i < E; i += 64) mx = fmaxf(mx, lg[i]);
  mx = wave_max(mx);
  const double m = mx;
  double sum = 0;
  for (int i = l; i < E; i += 64) sum = sum + exp((double)lg[i] - m);
  sum = wave_sum(sum, 64);
  for (int i = t; i < E; i += 256) {
    const float v = lg[i];
    const int rank = logit_rank(lg, E32, i, v);
    if (rank < K) {
      pw[rank] = (float)(exp((double)v - m) / sum);
      pid[rank] = i;
    }
  }
  __syncthreads();
  if (t < 64) {
    float wt = l < K ? pw[l] : 0.f;
    const int my_id = l < K ? pid[l] : 0x7fffffff;
    if (norm) {
      // the picked weights summed in pick order, as the reference's loop does
      double picked = 0;
      for (int j = 0; j < K; j++) picked = picked + (double)pw[j];
      wt = (float)((double)wt / picked);
    }
    // sorted by id: a pick's place is the number of smaller ids picked
    int place = 0;
    for (int j = 0; j < K; j++) place += pid[j] < my_id ? 1 : 0;
    if (l < K) {
      sid[place] = my_id;
      sw[place] = wt;
    }
  }
  __syncthreads();
}

}  // namespace ihip
