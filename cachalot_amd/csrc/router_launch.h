// Internal launcher of the router-score kernel (shared with the fused decode entry).
#pragma once

#include "common.h"

namespace cachalot {

// scores[t, e] = score_fn(dot(x[t], W[e]) / gate_temp) with the fixed reduction order
// (64 sequential chunks, xor butterfly).  Checks nothing: callers validate.
int launch_router_scores(const uint16_t* x, const uint16_t* W, int T, int D, int E, float gate_temp, int fn,
                         float* scores, hipStream_t s);

}  // namespace cachalot
