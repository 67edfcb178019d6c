// Pieces shared by the decode kernels (2-bit and FP4 banks).
#pragma once

#include "common.h"
#include "topk.h"

namespace cachalot {
namespace decode {

constexpr int KMAX = 8;     // max experts per token

struct Layout {
  int64_t record_bytes;
  int64_t off[9];
  bool f16;   // 2-bit banks: scales and biases stored as fp16 (else bf16)
};

inline int make_layout(const cachalot_expert_layout* layout, int n_tensors, const int* used, Layout& L,
                       const char* who) {
  L.record_bytes = layout->record_bytes;
  if (L.record_bytes <= 0 || L.record_bytes % 16 != 0)
    return fail(CACHALOT_EINVAL, "%s: record_bytes %lld must be a positive multiple of 16", who,
                (long long)L.record_bytes);
  for (int i = 0; i < 9; ++i) L.off[i] = layout->offset[i];
  if (layout->scale_dtype != CACHALOT_SCALE_BF16 && layout->scale_dtype != CACHALOT_SCALE_F16)
    return fail(CACHALOT_EINVAL, "%s: scale_dtype %d (0 = bf16, 1 = fp16)", who, (int)layout->scale_dtype);
  // FP4 records (six tensors) carry E8M0 scales: the flag has no meaning there
  if (n_tensors != 9 && layout->scale_dtype != CACHALOT_SCALE_BF16)
    return fail(CACHALOT_EINVAL, "%s: an FP4 bank has E8M0 scales, scale_dtype must be 0", who);
  L.f16 = layout->scale_dtype == CACHALOT_SCALE_F16;
  for (int t = 0; t < n_tensors; ++t) {
    const int i = used[t];
    if (L.off[i] < 0 || L.off[i] % 16 != 0 || L.off[i] >= L.record_bytes)
      return fail(CACHALOT_EINVAL, "%s: tensor offset %d (%lld) must be 16-byte aligned inside the record", who, i,
                  (long long)L.off[i]);
  }
  return CACHALOT_OK;
}

__device__ __forceinline__ float silu_f32(float g) { return g * (1.0f / (1.0f + expf(-g))); }

// Completion counters at the head of a decode workspace.  All are zero between
// calls: the router tail and the last down workgroup return them to zero.
struct Counters {
  unsigned int route_done;     // router workgroups finished (router tail)
  unsigned int gate_up_done;   // gate/up workgroups whose hidden rows are published
  unsigned int down_done;      // down workgroups finished
  unsigned int timeouts;       // waits that gave up (never expected; results then invalid)
};

// Upper bound on the polls of one wait (each poll sleeps ~64 clocks): a wait
// that has not seen its count by then gives up, so every wave always exits.
constexpr unsigned int SPIN_LIMIT = 1u << 22;

// Polls *c (agent-coherent loads) until it reaches `target`; false on timeout.
__device__ __forceinline__ bool wait_count(unsigned int* c, unsigned int target, unsigned int* timeouts) {
  for (unsigned int polls = 0; __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target; ++polls) {
    if (polls >= SPIN_LIMIT) {
      atomicAdd(timeouts, 1u);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// Agent-coherent 32-bit store (written through to the point every XCD reads from).
__device__ __forceinline__ void store_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void reset_counter(unsigned int* c) {
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Top-k tail of the router kernel (one token): the last workgroup to finish
// selects the experts, normalises their weights and resolves their slots.
struct RouteTail {
  const float* bias;
  const int32_t* slot_table;
  int32_t* idx_out;        // may be null
  float* w_out;            // may be null
  int32_t* ws_slots;       // [k] slot per routed expert (-1: not resident)
  float* ws_w;             // [k] router weight per routed expert
  unsigned int* counter;   // workgroups finished; zero between calls
  int E, k, order, norm;
  float route_scale;
};

// Workspace layout of one decode call:
//   [counters 256 B][k slots][k weights][hidden]
// each region 256-byte aligned, the counters at offset 0 whatever k and F are,
// so calls of different shapes on one workspace never overlap another's
// counters.  The counters must be zero before the first call on a workspace (a
// zero-filled allocation); every call leaves them zero.  The rest is scratch:
// nothing in it survives a call.
struct WsOffsets {
  size_t counter, slots, weights, hidden, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

inline WsOffsets ws_offsets(size_t hidden_bytes) {
  WsOffsets o;
  o.counter = 0;
  o.slots = 256;
  o.weights = o.slots + align256(KMAX * sizeof(int32_t));
  o.hidden = o.weights + align256(KMAX * sizeof(float));
  o.total = o.hidden + align256(hidden_bytes);
  return o;
}

// Where the expert kernels find routed expert e: given ids (idx != null: the
// slot comes from slot_table), the router's scores (scores != null: the gate/up
// kernels select the experts themselves, route_expert below) or the workspace's
// ws_slots / ws_w (written by whoever selected the experts).
struct ExpertSource {
  const int32_t* slot_table;
  const int32_t* idx;
  const float* w;
  int E;
  // selection from scores (router half of a layer-decode call)
  const float* scores;
  const float* bias;
  int k, order, norm;
  float route_scale;
  int32_t* idx_out;   // may be null
  float* w_out;       // may be null
};

__device__ __forceinline__ int expert_slot(const ExpertSource& src, const int32_t* ws_slots, int e) {
  if (src.idx) {
    const int ex = src.idx[e];
    return (ex >= 0 && ex < src.E) ? src.slot_table[ex] : -1;
  }
  return ws_slots[e];
}

__device__ __forceinline__ float expert_weight(const ExpertSource& src, const float* ws_w, int e) {
  return src.idx ? src.w[e] : ws_w[e];
}

// Slot of routed expert e, resolved by one whole wave.  With scores the wave
// runs the selection itself (the router's top-k, the same steps as
// router_topk_kernel), so no workgroup waits for another; lds_i / lds_v / lds_s
// are this wave's own KMAX-entry LDS arrays.  Every gate/up workgroup selects
// for itself and the results are identical.
__device__ __forceinline__ int route_slot(const ExpertSource& src, const int32_t* ws_slots, int e, int* lds_i,
                                          float* lds_v, int* lds_s) {
  if (src.scores == nullptr) return expert_slot(src, ws_slots, e);
  if (src.E <= 384) wave_topk<6>(src.scores, src.bias, src.E, src.k, src.order, lds_i, lds_v, src.slot_table, lds_s);
  else wave_topk<16>(src.scores, src.bias, src.E, src.k, src.order, lds_i, lds_v, src.slot_table, lds_s);
  return lds_s[e];
}

// Router weight of routed expert e (after route_slot; with scores, the
// normalisation of the selected scores by lane 0 into lds_w).
__device__ __forceinline__ float route_weight(const ExpertSource& src, const float* ws_w, int e, const float* lds_v,
                                              float* lds_w) {
  if (src.scores == nullptr) return expert_weight(src, ws_w, e);
  if ((threadIdx.x & 63) == 0) normalise_weights(lds_v, src.k, src.route_scale, src.norm, lds_w);
  return lds_w[e];
}

// Epilogue of a gate/up workgroup, lanes 0..15 of wave 0 (the wave whose LDS
// arrays route_slot filled): the router weight of expert e, also stored for the
// caller -- ws_w[e] by the expert's first tile, and the selection's ids and
// weights by the publishing workgroup.
__device__ __forceinline__ float route_finish(const ExpertSource& src, float* ws_w, int e, int tile,
                                              const float* lds_v, float* lds_w, const int* lds_i, bool publisher) {
  const float w = route_weight(src, ws_w, e, lds_v, lds_w);
  const int lane = threadIdx.x & 63;
  if (src.scores == nullptr) return w;
  if (tile == 0 && lane == 0) ws_w[e] = w;
  if (publisher && lane < src.k) {
    if (src.idx_out) src.idx_out[lane] = lds_i[lane];
    if (src.w_out) src.w_out[lane] = lds_w[lane];
  }
  return w;
}

}  // namespace decode
}  // namespace cachalot
