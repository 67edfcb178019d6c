// Expert-major permutation of up to THREADS routes by one workgroup of THREADS
// threads, thread i owning route i (E <= THREADS).  Counts per expert, their scan
// (offsets [E + 1]), then each route's row = its expert's offset + the number of
// earlier routes with the same key (the expert, or E for an id outside [0, E)), so
// rows stay in route order, as the reference assigns them
// (moe_prefill_grouped.py:199-225).  Dropped routes (key E) land after every expert
// with weight 0.
//
// Every thread reaches every barrier (no early return), so a kernel may go on to
// other work after the call; the rows and offsets are stored to global memory, and
// a __syncthreads() after the call makes them visible to the whole workgroup.
#pragma once

#include "common.h"

namespace cachalot {

template <int THREADS>
__device__ __forceinline__ void permute_small_body(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                   int n, int k, int E, int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ row_token, int32_t* __restrict__ row_slot,
                                                   float* __restrict__ row_w) {
  static_assert(THREADS % 64 == 0 && THREADS <= 1024, "one workgroup, whole waves");
  __shared__ int cnt[THREADS + 1];
  __shared__ int off[THREADS + 1];
  __shared__ __align__(16) int key[THREADS];
  __shared__ int wave_tot[THREADS / 64];
  const int i = threadIdx.x, lane = i & 63, wave = i >> 6;
  for (int e = i; e <= E; e += THREADS) cnt[e] = 0;
  const int id = i < n ? idx[i] : 0;
  const float wi = i < n ? w[i] : 0.0f;
  const int my = id >= 0 && id < E ? id : E;
  key[i] = i < n ? my : -1;
  __syncthreads();
  if (i < n && my < E) atomicAdd(&cnt[my], 1);
  __syncthreads();
  // exclusive scan of the counts: within the wave by shuffles, across waves by their totals
  const int c = i < E ? cnt[i] : 0;
  int v = c;
#pragma unroll
  for (int d = 1; d < 64; d *= 2) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  if (lane == 63) wave_tot[wave] = v;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int q = 0; q < THREADS / 64; ++q) {
    before += q < wave ? wave_tot[q] : 0;
    total += wave_tot[q];
  }
  if (i < E) {
    off[i] = before + v - c;
    offsets[i] = before + v - c;
  }
  if (i == 0) {
    off[E] = total;
    offsets[E] = total;
  }
  __syncthreads();
  if (i < n) {
    int rank = 0;
    const int4* k4 = reinterpret_cast<const int4*>(key);
    for (int j = 0; j < (i >> 2); ++j) {
      const int4 q = k4[j];
      rank += (q.x == my) + (q.y == my) + (q.z == my) + (q.w == my);
    }
    for (int j = i & ~3; j < i; ++j) rank += key[j] == my;
    const int pos = off[my] + rank;
    row_token[pos] = i / k;
    row_slot[pos] = i - (i / k) * k;
    row_w[pos] = my == E ? 0.0f : wi;
  }
}

}  // namespace cachalot
