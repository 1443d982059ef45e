// route.h - TDecoderModel.Route (decoder.pas:2901-2949) = route of
// ops.cu:664-720 as a block routine of 256 threads: softmax in double, the k
// highest logits (the lower id on a tie), weights rounded to single, renormed
// in pick order, then sorted by id. The pick order is a rank: logit i is the
// j-th pick when j logits are higher, or equal with a lower id; each thread
// counts it for its own logits against the row in LDS, eight 16-byte reads
// in flight. Used by the route kernel and inside the expert GEMV (which
// routes its token itself).
#pragma once

#include "common.h"

namespace ihip {

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
