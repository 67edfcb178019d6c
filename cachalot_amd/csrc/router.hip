// Router: logits -> score function -> biased top-k -> normalised weights.
//
// Reference semantics: src/cachalot/model/router_mlx.py:29-37 (DeepSeek),
// router_fused_metal.py:32-108 (fused kernels, tie rule), minimax/language.py:
// 280-292 and minimax/gpu_select.py:80-115 (sigmoid, rank order).
//
// Arithmetic contract (fixed so ids are reproducible bit for bit):
//   * D is cut into 16 contiguous chunks of D/16; 16 lanes own one chunk each
//     and add their bf16*bf16 products (exact in fp32) sequentially in fp32;
//   * the 16 partials are combined by an xor butterfly (8, 4, 2, 1);
//   * logit = sum / gate_temp (fp32);
//   * score functions use only IEEE basic operations (Cody-Waite exp with
//     a degree-13 Taylor polynomial, an atanh series for log1p), so a host
//     evaluation with the same steps agrees exactly;
//   * selection = score + bias; top-k by rank counting with the order's tie rule.
//
// Kernels
//   router_scores_kernel  one wave = 4 expert rows x up to TT tokens; W row chunks
//                         are loaded once per wave and reused for TT tokens.
//   router_topk_kernel    one workgroup per token; thread e computes the rank of
//                         expert e among all E by counting the experts that beat it.
#include "common.h"

namespace cachalot {
namespace {

constexpr int CHUNKS = 16;
constexpr int TT = 4;  // tokens per wave pass

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

// grid.x = ceil(E / (4 * waves)), grid.y = ceil(T / TT); block = 64 * waves
__global__ void __launch_bounds__(256) router_scores_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ W, int T, int D,
                                                            int E, float gate_temp, int fn,
                                                            float* __restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int row = (blockIdx.x * waves + wave) * 4 + (lane >> 4);
  const int chunk = lane & 15;
  const int t0 = blockIdx.y * TT;
  const int ch = D / CHUNKS;  // multiple of 8 (checked on the host)
  const bool row_ok = row < E;
  const uint4* wp = reinterpret_cast<const uint4*>(W + (size_t)(row_ok ? row : 0) * D + (size_t)chunk * ch);
  float acc[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) acc[j] = 0.0f;
  const uint4* xp[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const int t = min(t0 + j, T - 1);
    xp[j] = reinterpret_cast<const uint4*>(x + (size_t)t * D + (size_t)chunk * ch);
  }
  for (int v = 0; v < ch / 8; ++v) {
    const uint4 wv = wp[v];
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const uint4 xv = xp[j][v];
      const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[j] = acc[j] + __uint_as_float(xx[q] << 16) * __uint_as_float(ww[q] << 16);
        acc[j] = acc[j] + __uint_as_float(xx[q] & 0xffff0000u) * __uint_as_float(ww[q] & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TT; ++j) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) acc[j] = acc[j] + __shfl_xor(acc[j], m, 64);
  }
  if (chunk == 0 && row_ok) {
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int t = t0 + j;
      if (t < T) scores[(size_t)t * E + row] = score_of(acc[j] / gate_temp, fn);
    }
  }
}

// One workgroup (>= E threads, multiple of 64) per token.  Dynamic LDS holds
// the E selection values followed by the k winners' scores.
__global__ void __launch_bounds__(1024) router_topk_kernel(const float* __restrict__ scores,
                                                           const float* __restrict__ bias,
                                                           const float* __restrict__ bias_vl,
                                                           const uint8_t* __restrict__ image_mask, int E,
                                                           int k, float route_scale, int norm, int order,
                                                           int32_t* __restrict__ idx, float* __restrict__ w) {
  extern __shared__ float lds[];
  float* sel = lds;
  float* top = lds + E;
  const int t = blockIdx.x;
  const int e = threadIdx.x;
  const float* s = scores + (size_t)t * E;
  const float* b = (image_mask != nullptr && image_mask[t] != 0) ? bias_vl : bias;
  if (e < E) {
    float v = s[e] + b[e];
    if (v != v) v = -INFINITY;  // NaN never wins
    sel[e] = v;
  }
  __syncthreads();
  if (e < E) {
    const float me = sel[e];
    int rank = 0;
    if (order == CACHALOT_ORDER_ASCENDING) {
      // stable argsort(sel)[-k:]: a tie goes to the larger index
      for (int j = 0; j < E; ++j) {
        const float o = sel[j];
        rank += (o > me || (o == me && j > e)) ? 1 : 0;
      }
    } else {
      // argpartition(-sel): a tie goes to the lower index
      for (int j = 0; j < E; ++j) {
        const float o = sel[j];
        rank += (o > me || (o == me && j < e)) ? 1 : 0;
      }
    }
    if (rank < k) {
      const int pos = order == CACHALOT_ORDER_ASCENDING ? k - 1 - rank : rank;
      idx[(size_t)t * k + pos] = e;
      top[pos] = s[e];
    }
  }
  __syncthreads();
  if (e == 0) {
    float* wt = w + (size_t)t * k;
    if (norm && k > 1) {
      float total = 0.0f;
      for (int j = 0; j < k; ++j) total = total + top[j];
      const float denom = total + 1e-20f;
      for (int j = 0; j < k; ++j) wt[j] = (top[j] / denom) * route_scale;
    } else {
      for (int j = 0; j < k; ++j) wt[j] = top[j] * route_scale;
    }
  }
}

}  // namespace
}  // namespace cachalot

extern "C" int cachalot_router_topk(const uint16_t* x, const uint16_t* W, const float* bias,
                                    const float* bias_vl, const uint8_t* image_mask, int T, int D, int E,
                                    int k, int score_fn, float gate_temp, float route_scale, int norm,
                                    int order, int32_t* idx, float* w, float* scores,
                                    cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(x && W && bias && idx && w && scores, "router: null pointer");
  CACHALOT_REQUIRE(T >= 1, "router: x must contain at least one token (T=%d)", T);
  CACHALOT_REQUIRE(D >= 128 && D % 128 == 0, "router: D=%d must be a positive multiple of 128", D);
  CACHALOT_REQUIRE(E >= 1 && E <= 1024, "router: E=%d outside 1..1024", E);
  CACHALOT_REQUIRE(k >= 1 && k <= E, "router: invalid topk=%d for %d experts", k, E);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "router: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "router: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "router: gate_temp must be non-zero");
  CACHALOT_REQUIRE((image_mask == nullptr) == (bias_vl == nullptr),
                   "router: bias_vl and image_mask must be supplied together, or neither");
  hipStream_t s = (hipStream_t)stream;
  const int waves = 4;
  dim3 g1((E + 4 * waves - 1) / (4 * waves), (T + TT - 1) / TT);
  hipLaunchKernelGGL(router_scores_kernel, g1, dim3(64 * waves), 0, s, x, W, T, D, E, gate_temp, score_fn,
                     scores);
  int rc = check_launch("router_scores_kernel");
  if (rc) return rc;
  const int threads = ((E + 63) / 64) * 64;
  hipLaunchKernelGGL(router_topk_kernel, dim3(T), dim3(threads), (E + k) * sizeof(float), s, scores, bias, bias_vl,
                     image_mask, E, k, route_scale, norm, order, idx, w);
  return check_launch("router_topk_kernel");
}
