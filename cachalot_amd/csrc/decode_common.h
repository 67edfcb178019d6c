// Pieces shared by the decode kernels (2-bit and FP4 banks).
#pragma once

#include "common.h"
#include "topk.h"

namespace cachalot {
namespace decode {

constexpr int WAVES = 4;    // waves per workgroup
constexpr int R_DN = 2;     // W2 rows per wave in the down kernels
constexpr int KMAX = 8;     // max experts per token

struct Layout {
  int64_t record_bytes;
  int64_t off[9];
};

inline int make_layout(const cachalot_expert_layout* layout, int n_tensors, const int* used, Layout& L,
                       const char* who) {
  L.record_bytes = layout->record_bytes;
  if (L.record_bytes <= 0 || L.record_bytes % 16 != 0)
    return fail(CACHALOT_EINVAL, "%s: record_bytes %lld must be a positive multiple of 16", who,
                (long long)L.record_bytes);
  for (int i = 0; i < 9; ++i) L.off[i] = layout->offset[i];
  for (int t = 0; t < n_tensors; ++t) {
    const int i = used[t];
    if (L.off[i] < 0 || L.off[i] % 16 != 0 || L.off[i] >= L.record_bytes)
      return fail(CACHALOT_EINVAL, "%s: tensor offset %d (%lld) must be 16-byte aligned inside the record", who, i,
                  (long long)L.off[i]);
  }
  return CACHALOT_OK;
}

__device__ __forceinline__ int expert_slot(const int32_t* slot_table, const int32_t* idx, int e, int E) {
  const int ex = idx[e];
  if (ex < 0 || ex >= E) return -1;
  return slot_table[ex];
}

__device__ __forceinline__ float silu_f32(float g) { return g * (1.0f / (1.0f + expf(-g))); }

struct RouteArgs {            // fused top-k inputs (FUSE_TOPK)
  const float* scores;
  const float* bias;
  int E;
  int order;
  int norm;
  float route_scale;
  int32_t* idx_out;
  float* w_out;
};

// Workgroup prologue shared by the gate/up kernels of both banks: the k
// experts' slots and router weights into LDS; with FUSE the top-k itself.
template <bool FUSE>
__device__ __forceinline__ void expert_prologue(const int32_t* __restrict__ slot_table, const int32_t* __restrict__ idx,
                                                const float* __restrict__ wts, int E, int k, const RouteArgs& ra,
                                                int* s_slot, float* s_w, float4* sel4, int* top_i, float* top_v,
                                                int32_t* ws_slots, float* ws_w) {
  if constexpr (FUSE) {
    const int E4 = (ra.E + 3) / 4;
    load_selection(sel4, ra.E, E4, ra.scores, ra.bias);
    __syncthreads();
    block_topk_rank(sel4, ra.E, E4, k, ra.order, ra.scores, top_i, top_v);
    __syncthreads();
    if (threadIdx.x == 0) normalise_weights(top_v, k, ra.route_scale, ra.norm, s_w);
    if (threadIdx.x < k) {
      const int ex = top_i[threadIdx.x];
      s_slot[threadIdx.x] = slot_table[ex];
      if (blockIdx.x == 0 && ra.idx_out) ra.idx_out[threadIdx.x] = ex;
    }
    __syncthreads();
    if (blockIdx.x == 0 && threadIdx.x < k) {
      if (ra.w_out) ra.w_out[threadIdx.x] = s_w[threadIdx.x];
      ws_slots[threadIdx.x] = s_slot[threadIdx.x];
      ws_w[threadIdx.x] = s_w[threadIdx.x];
    }
  } else {
    if (threadIdx.x < k) {
      const int ex = idx[threadIdx.x];
      const int slot = (ex >= 0 && ex < E) ? slot_table[ex] : -1;
      s_slot[threadIdx.x] = slot;
      s_w[threadIdx.x] = wts[threadIdx.x];
      if (blockIdx.x == 0) {
        ws_slots[threadIdx.x] = slot;
        ws_w[threadIdx.x] = wts[threadIdx.x];
      }
    }
    __syncthreads();
  }
}

// Workspace layout of one decode call: [row-block counters][k slots][k weights]
// [hidden][per-expert row values], each region 256-byte aligned.  The counter
// region comes first and has a fixed size (enough for D <= MAX_D), so every
// call -- whatever its D, F, k or bank kind -- finds its counters at the same
// place.  It must be zero before the first call; every call leaves it zero.
constexpr int MAX_D = 8192;

struct WsOffsets {
  size_t counters, slots, weights, hidden, ybuf, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

inline WsOffsets ws_offsets(int D, int F, int k, size_t hidden_bytes) {
  (void)F;
  WsOffsets o;
  o.counters = 0;
  o.slots = align256((size_t)(MAX_D / R_DN) * sizeof(uint32_t));
  o.weights = o.slots + align256(KMAX * sizeof(int32_t));
  o.hidden = o.weights + align256(KMAX * sizeof(float));
  o.ybuf = o.hidden + align256(hidden_bytes);
  o.total = o.ybuf + align256((size_t)k * D * sizeof(float));
  return o;
}

// After wave_transpose_sum<R_DN>: row r's total sits in lanes [32r, 32r+32).
// Stores this expert's row values, then the last of the k waves of row block
// rb (device-scope counter) sums the k values in route order (bf16-rounded per
// expert when BF16_PER_EXPERT), adds the addend, writes the outputs and resets
// the counter for the next call.
template <bool BF16_PER_EXPERT>
__device__ __forceinline__ void combine_rows(float red, int lane, int e, int rb, int row0, int D, int k,
                                             float* __restrict__ ybuf, uint32_t* __restrict__ counters,
                                             const uint16_t* __restrict__ addend, float* __restrict__ routed,
                                             uint16_t* __restrict__ out) {
  static_assert(R_DN == 2, "lane mapping assumes two rows per wave");
  const float y = BF16_PER_EXPERT ? round_bf16(red) : red;
  const int n_own = row0 + (lane >> 5);
  if ((lane & 31) == 0 && n_own < D) ybuf[(size_t)e * D + n_own] = y;
  __threadfence();
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(&counters[rb], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  if (old != (uint32_t)(k - 1)) return;
  __threadfence();
  if (lane < R_DN && row0 + lane < D) {
    const int n = row0 + lane;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) {
      const uint32_t bits = __hip_atomic_load(reinterpret_cast<uint32_t*>(ybuf + (size_t)j * D + n),
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      acc = acc + __uint_as_float(bits);
    }
    if (routed) routed[n] = acc;
    if (out) out[n] = f32_to_bf16(addend ? acc + bf16_to_f32(addend[n]) : acc);
  }
  if (lane == 0) __hip_atomic_store(&counters[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace decode
}  // namespace cachalot
