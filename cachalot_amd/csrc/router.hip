// Router: logits -> score function -> biased top-k -> normalised weights.
//
// Reference semantics: src/cachalot/model/router_mlx.py:29-37 (DeepSeek),
// router_fused_metal.py:32-108 (fused kernels, tie rule), minimax/language.py:
// 280-292 and minimax/gpu_select.py:80-115 (sigmoid, rank order).
//
// Arithmetic contract (fixed so ids are reproducible bit for bit):
//   * D is cut into 64 contiguous chunks of D/64; lane l owns chunk l and adds
//     its bf16*bf16 products (exact in fp32) sequentially in fp32;
//   * the 64 partials are combined by the xor butterfly 1, 2, 4, 8, 16, 32
//     (pairwise summation over the chunks in natural order);
//   * logit = sum / gate_temp (fp32);
//   * score functions use only IEEE basic operations (Cody-Waite exp with
//     a degree-13 Taylor polynomial, an atanh series for log1p), so a host
//     evaluation with the same steps agrees exactly;
//   * selection = score + bias; top-k by rank counting with the order's tie rule.
//
// Kernels
//   router_scores_kernel  one wave = 4 expert rows x up to TT tokens; W row chunks
//                         are loaded once per wave and reused for TT tokens.
//   router_topk_kernel    one wave per token; k rounds of a wave-wide argmax
//                         under the order's total order (value, then index).
#include "mx_tile.h"
#include "router_launch.h"
#include "router_math.h"
#include "topk.h"

namespace cachalot {
namespace {

// Top-k tail for one token: every workgroup counts itself finished; the last one
// selects the experts (one wave), normalises the weights, resolves the slots and
// returns the counter to zero.  Protocol: the scores are stored with agent-scope
// (write-through) stores and each wave waits for its stores to complete before
// the workgroup counts itself with a returning agent-scope add; the selecting
// wave reads the scores with agent-scope loads.  (No release/acquire fences:
// those write back / invalidate whole L2s.)
__device__ __forceinline__ void route_tail(const float* __restrict__ scores, const decode::RouteTail& tail) {
  __shared__ int last;
  __shared__ int top_i[decode::KMAX], top_s[decode::KMAX];
  __shared__ float top_v[decode::KMAX];
  __shared__ float w[decode::KMAX];
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's score stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned done = __hip_atomic_fetch_add(tail.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = done == gridDim.x * gridDim.y - 1;
  }
  __syncthreads();
  if (!last || threadIdx.x >= 64) return;
  if (tail.E <= 384)
    wave_topk<6, true>(scores, tail.bias, tail.E, tail.k, tail.order, top_i, top_v, tail.slot_table, top_s);
  else
    wave_topk<16, true>(scores, tail.bias, tail.E, tail.k, tail.order, top_i, top_v, tail.slot_table, top_s);
  if (threadIdx.x == 0) normalise_weights(top_v, tail.k, tail.route_scale, tail.norm, w);
  if (threadIdx.x < tail.k) {
    tail.ws_slots[threadIdx.x] = top_s[threadIdx.x];
    tail.ws_w[threadIdx.x] = w[threadIdx.x];
    if (tail.idx_out) tail.idx_out[threadIdx.x] = top_i[threadIdx.x];
    if (tail.w_out) tail.w_out[threadIdx.x] = w[threadIdx.x];
  }
  if (threadIdx.x == 0) __hip_atomic_store(tail.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave per expert row (lane l owns chunk l of D/64 elements), TT tokens per
// wave, 4 waves per workgroup; optionally the top-k tail (one token).
template <int TT, int NV>
__global__ void __launch_bounds__(256) router_scores_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ W, int T, int D,
                                                            int E, float gate_temp, int fn,
                                                            float* __restrict__ scores, decode::RouteTail tail,
                                                            uint8_t* __restrict__ xplanes) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (xplanes != nullptr && blockIdx.y == 0) {   // token 0 as fp8 planes for the matrix-core decode
    for (int t4 = blockIdx.x * 256 + (int)threadIdx.x; 4 * t4 < D; t4 += gridDim.x * 256)
      mx::encode_x_quad(xplanes, t4, reinterpret_cast<const uint2*>(x)[t4]);   // whole quads of lanes
  }
  if (row < E) router_row<TT, NV>(x, W, T, D, E, gate_temp, fn, scores, row, lane, tail.counter != nullptr);
  if (tail.counter != nullptr) route_tail(scores, tail);
}

// One wave per token: k rounds of a wave-wide argmax (EPT = ceil(E / 64) candidates per lane).
template <int EPT>
__global__ void __launch_bounds__(64) router_topk_kernel(const float* __restrict__ scores,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ bias_vl,
                                                         const uint8_t* __restrict__ image_mask, int E, int k,
                                                         float route_scale, int norm, int order,
                                                         int32_t* __restrict__ idx, float* __restrict__ w) {
  __shared__ int top_i[1024];
  __shared__ float top_v[1024];
  const int t = blockIdx.x;
  const float* s = scores + (size_t)t * E;
  const float* b = (image_mask != nullptr && image_mask[t] != 0) ? bias_vl : bias;
  wave_topk<EPT>(s, b, E, k, order, top_i, top_v);
  __syncthreads();
  for (int j = threadIdx.x; j < k; j += 64) idx[(size_t)t * k + j] = top_i[j];
  if (threadIdx.x == 0) normalise_weights(top_v, k, route_scale, norm, w + (size_t)t * k);
}

}  // namespace

template <int TT>
static void launch_scores_tt(const uint16_t* x, const uint16_t* W, int T, int D, int E, float temp, int fn,
                             float* scores, hipStream_t s, const decode::RouteTail& tail, uint8_t* xplanes) {
  dim3 grid((E + 3) / 4, (T + TT - 1) / TT);
  switch (D) {
    case 4096: hipLaunchKernelGGL((router_scores_kernel<TT, 8>), grid, dim3(256), 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    case 5120: hipLaunchKernelGGL((router_scores_kernel<TT, 10>), grid, dim3(256), 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    case 7168: hipLaunchKernelGGL((router_scores_kernel<TT, 14>), grid, dim3(256), 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    default: hipLaunchKernelGGL((router_scores_kernel<TT, 0>), grid, dim3(256), 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
  }
}

int launch_router_scores(const uint16_t* x, const uint16_t* W, int T, int D, int E, float gate_temp, int fn,
                         float* scores, hipStream_t s, const decode::RouteTail* tail, uint8_t* xplanes) {
  decode::RouteTail none{};
  if (T >= 4) launch_scores_tt<4>(x, W, T, D, E, gate_temp, fn, scores, s, none, nullptr);
  else launch_scores_tt<1>(x, W, T, D, E, gate_temp, fn, scores, s, tail && T == 1 ? *tail : none, xplanes);
  return check_launch("router_scores_kernel");
}

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
  int rc = launch_router_scores(x, W, T, D, E, gate_temp, score_fn, scores, s);
  if (rc) return rc;
  if (E <= 384)
    hipLaunchKernelGGL((router_topk_kernel<6>), dim3(T), dim3(64), 0, s, scores, bias, bias_vl, image_mask, E, k,
                       route_scale, norm, order, idx, w);
  else
    hipLaunchKernelGGL((router_topk_kernel<16>), dim3(T), dim3(64), 0, s, scores, bias, bias_vl, image_mask, E, k,
                       route_scale, norm, order, idx, w);
  return check_launch("router_topk_kernel");
}
