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

int launch_router_scores(const uint16_t* x, const uint16_t* W, int T, int D, int E, float gate_temp, int fn,
                         float* scores, hipStream_t s, const decode::RouteTail* tail = nullptr);

}  // namespace cachalot
