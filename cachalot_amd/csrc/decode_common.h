// Pieces shared by the decode kernels (2-bit and FP4 banks).
#pragma once

#include "common.h"
#include "topk.h"

namespace cachalot {
namespace decode {

constexpr int WAVES = 4;    // waves per workgroup
constexpr int R_DN = 4;     // W2 rows per workgroup in the down kernels (one wave per expert)
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
                                                int* s_slot, float* s_w, int* top_i, float* top_v, float* lds_v,
                                                int* lds_i, int32_t* ws_slots, float* ws_w) {
  if constexpr (FUSE) {
    if (threadIdx.x < 64) {
      if (ra.E <= 384) wave_topk<6>(ra.scores, ra.bias, ra.E, k, ra.order, top_i, top_v);
      else wave_topk<16>(ra.scores, ra.bias, ra.E, k, ra.order, top_i, top_v);
    }
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

// Workspace layout of one decode call: [k slots][k weights][hidden], each
// region 256-byte aligned.  Scratch only: nothing in it survives a call.
struct WsOffsets {
  size_t slots, weights, hidden, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

inline WsOffsets ws_offsets(size_t hidden_bytes) {
  WsOffsets o;
  o.slots = 0;
  o.weights = align256(KMAX * sizeof(int32_t));
  o.hidden = o.weights + align256(KMAX * sizeof(float));
  o.total = o.hidden + align256(hidden_bytes);
  return o;
}

// Row r's total sits in lanes [16r, 16r+16) after wave_transpose_sum<R_DN>.
// Each of the k waves of the workgroup (wave e = expert e) leaves its row values
// in LDS; after the barrier the first R_DN threads sum the k values of their row
// in route order (each bf16-rounded when BF16_PER_EXPERT), add the addend and
// write the outputs.
template <bool BF16_PER_EXPERT>
__device__ __forceinline__ void combine_rows(float red, int lane, int e, int row0, int D, int k,
                                             float (*vals)[R_DN], const uint16_t* __restrict__ addend,
                                             float* __restrict__ routed, uint16_t* __restrict__ out) {
  static_assert(R_DN == 4, "lane mapping assumes four rows per workgroup");
  if ((lane & 15) == 0) vals[e][lane >> 4] = BF16_PER_EXPERT ? round_bf16(red) : red;
  __syncthreads();
  const int t = threadIdx.x;
  if (t < R_DN && row0 + t < D) {
    const int n = row0 + t;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) acc = acc + vals[j][t];
    if (routed) routed[n] = acc;
    if (out) out[n] = f32_to_bf16(addend ? acc + bf16_to_f32(addend[n]) : acc);
  }
}

}  // namespace decode
}  // namespace cachalot
