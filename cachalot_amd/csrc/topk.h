// Top-k over E selection values (score + bias) by one wave, shared by the
// router kernels and the decode gate/up prologue.
//
// Order: value, then index -- ascending order (stable argsort(sel)[-k:]) gives a
// tie to the larger index, rank order (argpartition(-sel)) to the lower one;
// NaN never wins (it ranks as -inf) and -0 ties with +0, as float comparison
// has it.  Each value becomes an order-preserving u32 key, so one round is a
// u32 max over the lane's EPT keys and over the wave (DPP), then the index rule
// on the ballots of the maximum's holders, and the winner's owner clears its key.
#pragma once

#include "common.h"

namespace cachalot {

// Order-preserving key of a selection value (0 is below every value's key and
// marks candidates that can no longer win).
__device__ __forceinline__ uint32_t topk_key(float s) {
  if (s != s) s = -INFINITY;
  s = s + 0.0f;   // -0 -> +0
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// u32 max over the wave, returned to every lane (uniform): the row maxima by four
// DPP steps (every lane of a row of 16 ends with its row's maximum), then the
// row broadcasts 15 and 31 carry rows 0-1 into rows 1-3, so lane 63 holds the
// maximum of all four rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t m) {
  m = max(m, xor1_u32(m));
  m = max(m, xor2_u32(m));
  m = max(m, mirror8_u32(m));
  m = max(m, mirror16_u32(m));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x142, 0xa, 0xf, false));   // row_bcast:15
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x143, 0xc, 0xf, false));   // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
}

// Writes top_i[pos] / top_v[pos] (winner index and its raw score), pos = k-1-r
// (ascending order) or r (rank order) for round r, and, with a slot table,
// top_s[pos] = slot_table[winner] (the table is read with the scores, so the
// slot costs no dependent load).  COHERENT: the scores are read with agent-scope
// loads (written by other workgroups of the running kernel).  Requires
// E <= 64 * EPT and 1 <= k <= E.
//
// A round: the wave maximum of the keys, then one ballot per key register of the
// holders of that maximum; the winner is found from the ballots with scalar bit
// scans -- the highest index holding it (ascending order) or the lowest (rank
// order) -- so ties cost nothing extra, and its owner clears its key.
template <int EPT, bool COHERENT = false>
__device__ __forceinline__ void wave_topk(const float* __restrict__ scores, const float* __restrict__ bias, int E,
                                          int k, int order, int* top_i, float* top_v,
                                          const int32_t* __restrict__ slot_table = nullptr, int* top_s = nullptr) {
  const int lane = threadIdx.x & 63;
  // unconditional (clamped) loads, so all of them are in flight together
  float sv[EPT], bv0[EPT];
  int st[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = min(lane + 64 * j, E - 1);
    sv[j] = COHERENT ? __hip_atomic_load(&scores[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : scores[e];
    bv0[j] = bias[e];
    st[j] = slot_table ? slot_table[e] : 0;
  }
  uint32_t key[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) key[j] = lane + 64 * j < E ? topk_key(sv[j] + bv0[j]) : 0u;
  const bool asc = order == CACHALOT_ORDER_ASCENDING;
  for (int r = 0; r < k; ++r) {
    uint32_t m = key[0];
#pragma unroll
    for (int j = 1; j < EPT; ++j) m = max(m, key[j]);
    const uint32_t mu = wave_max_u32(m);
    uint64_t hold[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) hold[j] = __ballot(key[j] == mu);
    int win = -1;
    if (asc) {
#pragma unroll
      for (int j = EPT - 1; j >= 0; --j)
        if (win < 0 && hold[j] != 0) win = 64 * j + 63 - __clzll((long long)hold[j]);
    } else {
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        if (win < 0 && hold[j] != 0) win = 64 * j + __ffsll((long long)hold[j]) - 1;
    }
    win = __builtin_amdgcn_readfirstlane(win);
    const int wl = win & 63, wj = win >> 6;
#pragma unroll
    for (int j = 0; j < EPT; ++j) key[j] = (j == wj && lane == wl) ? 0u : key[j];
    if (lane == 0) top_i[asc ? k - 1 - r : r] = win;
  }
  // position p (lane p % 64): the raw score (and slot) of winner top_i[p], fetched from its owner lane
  for (int p0 = 0; p0 < k; p0 += 64) {
    const int p = p0 + lane;
    const int wi = p < k ? top_i[p] : 0;
    float sw = 0.0f;
    int ss = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const float vj = __shfl(sv[j], wi & 63, 64);
      const int tj = __shfl(st[j], wi & 63, 64);
      sw = (wi >> 6) == j ? vj : sw;
      ss = (wi >> 6) == j ? tj : ss;
    }
    if (p < k) {
      top_v[p] = sw;
      if (top_s) top_s[p] = ss;
    }
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
