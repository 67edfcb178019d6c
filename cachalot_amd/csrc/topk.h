// Block-wide top-k over E selection values, shared by the router kernel and
// the fused decode prologue.
//
// Rank counting: thread e owns expert e and counts the experts that beat it
// under the order's total order (value, then index: ascending order = stable
// argsort(sel)[-k:], a tie goes to the larger index; rank order =
// argpartition(-sel), a tie goes to the lower index).  Ranks are a
// permutation, so exactly k threads write, each to its own output position.
// The E values sit in LDS padded with -inf to a multiple of 4 and are read
// back as float4 broadcasts.
#pragma once

#include "common.h"

namespace cachalot {

// sel4: LDS, E4 = ceil(E/4) float4 (padding -inf); out_idx/out_val: LDS [k]
__device__ __forceinline__ void block_topk_rank(const float4* __restrict__ sel4, int E, int E4, int k, int order,
                                                const float* __restrict__ scores, int* out_idx, float* out_val) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const float* sel = reinterpret_cast<const float*>(sel4);
    const float me = sel[e];
    int rank = 0;
    if (order == CACHALOT_ORDER_ASCENDING) {
#pragma unroll 8
      for (int j4 = 0; j4 < E4; ++j4) {
        const float4 o = sel4[j4];
        const int j = 4 * j4;
        rank += (o.x > me || (o.x == me && j > e)) ? 1 : 0;
        rank += (o.y > me || (o.y == me && j + 1 > e)) ? 1 : 0;
        rank += (o.z > me || (o.z == me && j + 2 > e)) ? 1 : 0;
        rank += (o.w > me || (o.w == me && j + 3 > e)) ? 1 : 0;
      }
    } else {
#pragma unroll 8
      for (int j4 = 0; j4 < E4; ++j4) {
        const float4 o = sel4[j4];
        const int j = 4 * j4;
        rank += (o.x > me || (o.x == me && j < e)) ? 1 : 0;
        rank += (o.y > me || (o.y == me && j + 1 < e)) ? 1 : 0;
        rank += (o.z > me || (o.z == me && j + 2 < e)) ? 1 : 0;
        rank += (o.w > me || (o.w == me && j + 3 < e)) ? 1 : 0;
      }
    }
    if (rank < k) {
      const int pos = order == CACHALOT_ORDER_ASCENDING ? k - 1 - rank : rank;
      out_idx[pos] = e;
      out_val[pos] = scores[e];
    }
  }
}

// a beats b under the order's total order; an index < 0 marks "no candidate".
__device__ __forceinline__ bool topk_better(float a, int ai, float b, int bi, int order) {
  if (ai < 0) return false;
  if (bi < 0) return true;
  if (a != b) return a > b;
  return order == CACHALOT_ORDER_ASCENDING ? ai > bi : ai < bi;
}

// k rounds of a block-wide argmax (O(E) work per round): each thread keeps up
// to EPT candidates, a wave butterfly finds the wave's best, LDS holds one
// entry per wave, every thread derives the same block winner, the owner marks
// it taken.  Round r yields rank r.  Requires E <= EPT * blockDim.x and
// blockDim.x a multiple of 64 (<= 1024).  lds_v / lds_i: LDS [16].
template <int EPT>
__device__ __forceinline__ void block_topk_rounds(const float* __restrict__ scores, const float* __restrict__ bias,
                                                  int E, int k, int order, int* top_i, float* top_v, float* lds_v,
                                                  int* lds_i) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int nwaves = blockDim.x >> 6;
  float v[EPT];
  int id[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = tid + j * blockDim.x;
    id[j] = -1;
    v[j] = -INFINITY;
    if (e < E) {
      float s = scores[e] + bias[e];
      if (s != s) s = -INFINITY;  // NaN never wins
      v[j] = s;
      id[j] = e;
    }
  }
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = -1;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
      if (topk_better(v[j], id[j], bv, bi, order)) {
        bv = v[j];
        bi = id[j];
      }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(bv, m, 64);
      const int oi = __shfl_xor(bi, m, 64);
      if (topk_better(ov, oi, bv, bi, order)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      lds_v[tid >> 6] = bv;
      lds_i[tid >> 6] = bi;
    }
    __syncthreads();
    float wv = lds_v[0];
    int wi = lds_i[0];
    for (int w = 1; w < nwaves; ++w)
      if (topk_better(lds_v[w], lds_i[w], wv, wi, order)) {
        wv = lds_v[w];
        wi = lds_i[w];
      }
#pragma unroll
    for (int j = 0; j < EPT; ++j)
      if (id[j] == wi) id[j] = -1;
    if (tid == 0) {
      const int pos = order == CACHALOT_ORDER_ASCENDING ? k - 1 - r : r;
      top_i[pos] = wi;
      top_v[pos] = scores[wi];
    }
    __syncthreads();
  }
}

// Fill sel4 from scores + bias (NaN -> -inf, padding -inf).
__device__ __forceinline__ void load_selection(float4* sel4, int E, int E4, const float* __restrict__ scores,
                                               const float* __restrict__ bias) {
  float* sel = reinterpret_cast<float*>(sel4);
  for (int e = threadIdx.x; e < 4 * E4; e += blockDim.x) {
    float v = -INFINITY;
    if (e < E) {
      v = scores[e] + bias[e];
      if (v != v) v = -INFINITY;  // NaN never wins
    }
    sel[e] = v;
  }
}

// w_j = top_j / (sum_j top_j + 1e-20) * route_scale, sum in output order (norm and k > 1),
// else top_j * route_scale.  Single-threaded by design: the order of the sum is the contract.
__device__ __forceinline__ void normalise_weights(const float* top, int k, float route_scale, int norm, float* w) {
  if (norm && k > 1) {
    float total = 0.0f;
    for (int j = 0; j < k; ++j) total = total + top[j];
    const float denom = total + 1e-20f;
    for (int j = 0; j < k; ++j) w[j] = (top[j] / denom) * route_scale;
  } else {
    for (int j = 0; j < k; ++j) w[j] = top[j] * route_scale;
  }
}

}  // namespace cachalot
