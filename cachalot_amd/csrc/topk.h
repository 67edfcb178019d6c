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
  const bool idx_wins = order == CACHALOT_ORDER_ASCENDING ? ai > bi : ai < bi;
  return (ai >= 0) & ((bi < 0) | (a > b) | ((a == b) & idx_wins));
}

template <int M>
__device__ __forceinline__ void topk_exchange_step(float& bv, int& bi, int order) {
  float ov;
  int oi;
  if constexpr (M == 7) {
    ov = __uint_as_float(mirror8_u32(__float_as_uint(bv)));
    oi = (int)mirror8_u32((uint32_t)bi);
  } else if constexpr (M == 15) {
    ov = __uint_as_float(mirror16_u32(__float_as_uint(bv)));
    oi = (int)mirror16_u32((uint32_t)bi);
  } else {
    ov = xor_f<M>(bv);
    oi = (int)xor_u32<M>((uint32_t)bi);
  }
  const bool take = topk_better(ov, oi, bv, bi, order);
  bv = take ? ov : bv;
  bi = take ? oi : bi;
}

// Top-k by one wave: k rounds of a wave-wide argmax under the order's total
// order (a max-reduction, so the exchange pattern does not change the result),
// the winner's owner marks it taken.  Round r yields rank r.  Lane 0 writes
// top_i / top_v (LDS or global).  Requires E <= 64 * EPT.
template <int EPT>
__device__ __forceinline__ void wave_topk(const float* __restrict__ scores, const float* __restrict__ bias, int E,
                                          int k, int order, int* top_i, float* top_v) {
  const int lane = threadIdx.x & 63;
  float v[EPT];
  int id[EPT];
  // unconditional (clamped) loads, so all of them are in flight together
  float sv[EPT], bv0[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = min(lane + 64 * j, E - 1);
    sv[j] = scores[e];
    bv0[j] = bias[e];
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = lane + 64 * j;
    float s = sv[j] + bv0[j];
    if (s != s) s = -INFINITY;  // NaN never wins
    v[j] = s;
    id[j] = e < E ? e : -1;
  }
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = -1;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const bool take = topk_better(v[j], id[j], bv, bi, order);
      bv = take ? v[j] : bv;
      bi = take ? id[j] : bi;
    }
    topk_exchange_step<1>(bv, bi, order);
    topk_exchange_step<2>(bv, bi, order);
    topk_exchange_step<7>(bv, bi, order);
    topk_exchange_step<15>(bv, bi, order);
    topk_exchange_step<16>(bv, bi, order);
    topk_exchange_step<32>(bv, bi, order);
#pragma unroll
    for (int j = 0; j < EPT; ++j) id[j] = id[j] == bi ? -1 : id[j];
    if (lane == 0) {
      const int pos = order == CACHALOT_ORDER_ASCENDING ? k - 1 - r : r;
      top_i[pos] = bi;
    }
  }
  // the raw scores of the winners (the weights are taken from scores, not selection values)
  for (int j = lane; j < k; j += 64) top_v[j] = scores[top_i[j]];
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
