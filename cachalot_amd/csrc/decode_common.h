// Pieces shared by the decode kernels (2-bit and FP4 banks).
#pragma once

#include "common.h"

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

// After wave_transpose_sum<R_DN * KMAX>: value r*KMAX + e sits in lanes [4(r*KMAX+e), +4).
// Sums the k expert values of each row in route order (bf16-rounded per expert
// when BF16_PER_EXPERT), adds the addend and writes the requested outputs.
template <bool BF16_PER_EXPERT>
__device__ __forceinline__ void finish_rows(const float red, int lane, int row0, int D, int k,
                                            const uint16_t* __restrict__ addend, float* __restrict__ routed,
                                            uint16_t* __restrict__ out) {
  static_assert(R_DN * KMAX == 16, "lane mapping assumes 16 reduced values");
  float v[KMAX];
#pragma unroll
  for (int e = 0; e < KMAX; ++e) v[e] = __shfl(red, (lane & ~31) + 4 * e, 64);
  if ((lane & 31) == 0) {
    const int n = row0 + (lane >> 5);
    if (n < D) {
      float acc = 0.0f;
      for (int e = 0; e < k; ++e) acc = acc + (BF16_PER_EXPERT ? round_bf16(v[e]) : v[e]);
      if (routed) routed[n] = acc;
      if (out) {
        const float t = addend ? acc + bf16_to_f32(addend[n]) : acc;
        out[n] = f32_to_bf16(t);
      }
    }
  }
}

}  // namespace decode
}  // namespace cachalot
