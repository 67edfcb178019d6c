// Internal launcher of the router-score kernel (shared with the fused decode entry).
#pragma once

#include "common.h"
#include "decode_common.h"

namespace cachalot {

// scores[t, e] = score_fn(dot(x[t], W[e]) / gate_temp) with the fixed reduction order
// (64 sequential chunks, xor butterfly).  With `tail` (T == 1 only) the last
// workgroup to finish also runs the top-k tail (selection, weights, slots).
// Checks nothing: callers validate.
// The router half of a fused layer-decode call (one token).
struct RouterCall {
  const uint16_t* gate_weight;
  int score_fn;
  float gate_temp;
  float* scores;
  decode::RouteTail tail;
};

// The expert source of a layer-decode call whose gate/up kernels select the
// experts from the router's scores.
inline decode::ExpertSource route_source(const decode::ExpertSource& base, const RouterCall& r) {
  decode::ExpertSource src = base;
  src.idx = nullptr;
  src.w = nullptr;
  src.scores = r.scores;
  src.bias = r.tail.bias;
  src.k = r.tail.k;
  src.order = r.tail.order;
  src.norm = r.tail.norm;
  src.route_scale = r.tail.route_scale;
  src.idx_out = r.tail.idx_out;
  src.w_out = r.tail.w_out;
  return src;
}

// With xplanes (T == 1, D a multiple of 16) the kernel also writes x as fp8 plane
// blocks (mx_tile.h) for the matrix-core decode.
int launch_router_scores(const uint16_t* x, const uint16_t* W, int T, int D, int E, float gate_temp, int fn,
                         float* scores, hipStream_t s, const decode::RouteTail* tail = nullptr,
                         uint8_t* xplanes = nullptr);

}  // namespace cachalot
