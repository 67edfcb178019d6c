// Router score arithmetic shared by the router kernels and the decode kernels
// that score the experts themselves.  The contract (fixed so expert ids are
// reproducible bit for bit; reference: src/cachalot/model/router_mlx.py:29-37,
// minimax/language.py:280-292):
//   * D is cut into 64 contiguous chunks of D/64; lane l owns chunk l and adds
//     its bf16*bf16 products sequentially in fp32 with fma.  A product of two bf16
//     values has 16 significant bits, so it is exact in fp32 unless it falls below
//     the normal range (|x w| < 2^-126); then a multiply-then-add rounds it and the
//     fma does not, and the two can differ in the last bit.  Activations and gate
//     weights of a real layer (|x|, |w| far above 2^-63) never come near that;
//     the CPU restatement multiplies then adds;
//   * the 64 partials are combined by the xor butterfly 1, 2, 4, 8, 16, 32;
//   * logit = sum / gate_temp (fp32);
//   * score functions use only IEEE basic operations (Cody-Waite exp with a
//     degree-13 Taylor polynomial, an atanh series for log1p).
#pragma once

#include "common.h"

namespace cachalot {
namespace {

constexpr int CHUNKS = 64;  // one chunk per lane of a wave64

constexpr double INV_LN2 = 1.4426950408889634;
constexpr double LN2_HI = 6.93147180369123816490e-01;
constexpr double LN2_LO = 1.90821492927058770002e-10;
// 1/k!, k = 0..13 (correctly rounded doubles)
__constant__ double EXP_COEF[14] = {
    1.0, 1.0, 0.5, 0.16666666666666666, 0.041666666666666664, 0.008333333333333333,
    0.001388888888888889, 0.0001984126984126984, 2.48015873015873e-05, 2.7557319223985893e-06,
    2.755731922398589e-07, 2.505210838544172e-08, 2.08767569878681e-09, 1.6059043836821613e-10};
// 2/(2j+1), j = 0..16
__constant__ double LOG1P_COEF[17] = {
    2.0, 0.6666666666666666, 0.4, 0.2857142857142857, 0.2222222222222222, 0.18181818181818182,
    0.15384615384615385, 0.13333333333333333, 0.11764705882352941, 0.10526315789473684,
    0.09523809523809523, 0.08695652173913043, 0.08, 0.07407407407407407, 0.06896551724137931,
    0.06451612903225806, 0.06060606060606061};

__device__ double exp64(double a) {  // a <= 0
  if (a < -200.0) return 0.0;
  const double n = rint(a * INV_LN2);
  const double r = (a - n * LN2_HI) - n * LN2_LO;
  double p = EXP_COEF[13];
#pragma unroll
  for (int k = 12; k >= 0; --k) p = p * r + EXP_COEF[k];
  return ldexp(p, (int)n);
}

__device__ double log1p64(double t) {  // 0 <= t <= 1
  const double u = t / (2.0 + t);
  const double u2 = u * u;
  double q = LOG1P_COEF[16];
#pragma unroll
  for (int j = 15; j >= 0; --j) q = q * u2 + LOG1P_COEF[j];
  return u * q;
}

__device__ float score_of(float z32, int fn) {
  const double z = (double)z32;
  const double t = exp64(-fabs(z));
  if (fn == CACHALOT_SCORE_SIGMOID) {
    const float t32 = (float)t;
    return z32 >= 0.0f ? 1.0f / (1.0f + t32) : t32 / (1.0f + t32);
  }
  const double sp = fmax(z, 0.0) + log1p64(t);
  return sqrtf((float)sp);
}

// Score of one expert row: lane l owns chunk l of D/64 elements, TT tokens.
// NV = uint4 loads per lane per row (D = 512 * NV); NV = 0 is the generic path
// (D a multiple of 128, u32 loads).
template <int TT, int NV>
__device__ __forceinline__ void router_row(const uint16_t* __restrict__ x, const uint16_t* __restrict__ W, int T,
                                           int D, int E, float gate_temp, int fn, float* __restrict__ scores,
                                           int row, int lane, bool coherent) {
  const int t0 = blockIdx.y * TT;
  const int ch = D / CHUNKS;
  const uint16_t* wrow = W + (size_t)row * D + (size_t)lane * ch;
  const uint16_t* xrow[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) xrow[j] = x + (size_t)min(t0 + j, T - 1) * D + (size_t)lane * ch;
  float acc[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) acc[j] = 0.0f;
  if constexpr (NV > 0) {
    uint4 wv[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) wv[v] = reinterpret_cast<const uint4*>(wrow)[v];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      uint4 xv[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) xv[v] = reinterpret_cast<const uint4*>(xrow[j])[v];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const uint32_t ww[4] = {wv[v].x, wv[v].y, wv[v].z, wv[v].w};
        const uint32_t xx[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[j] = __builtin_fmaf(__uint_as_float(xx[q] << 16), __uint_as_float(ww[q] << 16), acc[j]);
          acc[j] = __builtin_fmaf(__uint_as_float(xx[q] & 0xffff0000u), __uint_as_float(ww[q] & 0xffff0000u), acc[j]);
        }
      }
    }
  } else {
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(wrow);
    for (int v = 0; v < ch / 2; ++v) {
      const uint32_t ww = wp[v];
#pragma unroll
      for (int j = 0; j < TT; ++j) {
        const uint32_t xx = reinterpret_cast<const uint32_t*>(xrow[j])[v];
        acc[j] = __builtin_fmaf(__uint_as_float(xx << 16), __uint_as_float(ww << 16), acc[j]);
        acc[j] = __builtin_fmaf(__uint_as_float(xx & 0xffff0000u), __uint_as_float(ww & 0xffff0000u), acc[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TT; ++j) acc[j] = wave_sum(acc[j]);
  if (lane < TT) {
    // lane j finishes token j (all lanes hold every total after the butterfly)
    float v = acc[0];
#pragma unroll
    for (int j = 1; j < TT; ++j)
      if (lane == j) v = acc[j];
    const int t = t0 + lane;
    if (t < T) {
      const float sc = score_of(v / gate_temp, fn);
      // with the top-k tail, stored through to where every XCD reads (see route_tail)
      if (coherent) __hip_atomic_store(&scores[(size_t)t * E + row], sc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else scores[(size_t)t * E + row] = sc;
    }
  }
}

}  // namespace
}  // namespace cachalot
