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

// Many tokens: one 256-thread workgroup = 32 tokens x 64 experts, each thread 2
// tokens x 4 experts.  The same arithmetic as router_row: chunk c (of 64) of every
// dot product is a sequential fp32 sum of its D/64 products, and the 64 chunk sums
// meet in the pairwise tree (left + right) the xor butterfly forms.  Chunk by chunk,
// x and W slices are staged in LDS as fp32; the tree is kept as a binary-counter
// stack of six partial nodes per dot product.  fma(x, w, s) equals s + x * w here:
// the product of two bf16 values is exact in fp32 (16 significant bits) unless it is
// below 2^-133 in magnitude.
constexpr int RT_T = 32;             // tokens per workgroup
constexpr int RT_E = 64;             // experts per workgroup
constexpr int RT_MAXCH = 80;         // D / 64 <= 80 (D <= 5120)
constexpr int RT_PAD = 4;            // floats of padding per staged row (bank spread)
constexpr int RT_MIN_T = 1024;       // fewer tokens: the 4-token kernel fills the chip better

__global__ void __launch_bounds__(256) router_tiled_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ W, int T, int D, int E,
                                                           float gate_temp, int fn, float* __restrict__ scores) {
  __shared__ __align__(16) float xs[RT_T][RT_MAXCH + RT_PAD];
  __shared__ __align__(16) float ws[RT_E][RT_MAXCH + RT_PAD];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int eq = lane & 15;                   // experts 4 eq .. 4 eq + 3
  const int tp = (lane >> 4) + 4 * wave;      // tokens 2 tp, 2 tp + 1
  const int t0 = blockIdx.x * RT_T, e0 = blockIdx.y * RT_E;
  const int ch = D / CHUNKS;                  // a multiple of 8
  const int xq = RT_T * ch / 8, wq = RT_E * ch / 8;   // 8-value items per chunk
  // staging: item -> (row, 8 values); rows past T / E read row 0 (results unused)
  auto load_chunk = [&](int c, uint4 (&xv)[2], uint4 (&wv)[3]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int it = tid + 256 * j;
      const int r = it / (ch / 8), q = it - r * (ch / 8);
      const int t = min(t0 + r, T - 1);
      xv[j] = it < xq ? *reinterpret_cast<const uint4*>(x + (size_t)t * D + c * ch + 8 * q) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int it = tid + 256 * j;
      const int r = it / (ch / 8), q = it - r * (ch / 8);
      const int e = min(e0 + r, E - 1);
      wv[j] = it < wq ? *reinterpret_cast<const uint4*>(W + (size_t)e * D + c * ch + 8 * q) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_chunk = [&](const uint4 (&xv)[2], const uint4 (&wv)[3]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int it = tid + 256 * j;
      if (it < xq) {
        const int r = it / (ch / 8), q = it - r * (ch / 8);
        const uint32_t u[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        float4* d = reinterpret_cast<float4*>(&xs[r][8 * q]);
        d[0] = make_float4(__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xffff0000u),
                           __uint_as_float(u[1] << 16), __uint_as_float(u[1] & 0xffff0000u));
        d[1] = make_float4(__uint_as_float(u[2] << 16), __uint_as_float(u[2] & 0xffff0000u),
                           __uint_as_float(u[3] << 16), __uint_as_float(u[3] & 0xffff0000u));
      }
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int it = tid + 256 * j;
      if (it < wq) {
        const int r = it / (ch / 8), q = it - r * (ch / 8);
        const uint32_t u[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
        float4* d = reinterpret_cast<float4*>(&ws[r][8 * q]);
        d[0] = make_float4(__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xffff0000u),
                           __uint_as_float(u[1] << 16), __uint_as_float(u[1] & 0xffff0000u));
        d[1] = make_float4(__uint_as_float(u[2] << 16), __uint_as_float(u[2] & 0xffff0000u),
                           __uint_as_float(u[3] << 16), __uint_as_float(u[3] & 0xffff0000u));
      }
    }
  };
  float stk[6][8];
  float node[8];
  uint4 xv[2], wv[3];
  load_chunk(0, xv, wv);
  store_chunk(xv, wv);
  __syncthreads();
  for (int c = 0; c < CHUNKS; ++c) {
    if (c + 1 < CHUNKS) load_chunk(c + 1, xv, wv);
    float acc[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) acc[p] = 0.0f;
    for (int k = 0; k < ch; k += 4) {
      float4 xa[2], wa[4];
#pragma unroll
      for (int a = 0; a < 2; ++a) xa[a] = *reinterpret_cast<const float4*>(&xs[2 * tp + a][k]);
#pragma unroll
      for (int b = 0; b < 4; ++b) wa[b] = *reinterpret_cast<const float4*>(&ws[4 * eq + b][k]);
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float v = acc[4 * a + b];
          v = __builtin_fmaf(xa[a].x, wa[b].x, v);
          v = __builtin_fmaf(xa[a].y, wa[b].y, v);
          v = __builtin_fmaf(xa[a].z, wa[b].z, v);
          v = __builtin_fmaf(xa[a].w, wa[b].w, v);
          acc[4 * a + b] = v;
        }
    }
    // merge chunk c into the tree (c is uniform: every branch below is too)
#pragma unroll
    for (int p = 0; p < 8; ++p) node[p] = acc[p];
    // chunk c closes the nodes of the levels below its lowest zero bit
    const int up = __builtin_ctz(~c);   // levels merged (6 after the last chunk)
#pragma unroll
    for (int L = 0; L < 6; ++L) {
      if (L < up) {
#pragma unroll
        for (int p = 0; p < 8; ++p) node[p] = stk[L][p] + node[p];
      } else if (L == up) {
#pragma unroll
        for (int p = 0; p < 8; ++p) stk[L][p] = node[p];
      }
    }
    __syncthreads();
    if (c + 1 < CHUNKS) {
      store_chunk(xv, wv);
      __syncthreads();
    }
  }
  // after chunk 63 every level merged: node holds the root
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int t = t0 + 2 * tp + a;
    if (t >= T) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int e = e0 + 4 * eq + b;
      if (e < E) scores[(size_t)t * E + e] = score_of(node[4 * a + b] / gate_temp, fn);
    }
  }
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
  // the tiled kernel needs enough tiles to fill the chip (32 x 64 per workgroup)
  if (T >= RT_MIN_T && D % 512 == 0 && D / CHUNKS <= RT_MAXCH) {
    hipLaunchKernelGGL(router_tiled_kernel, dim3((T + RT_T - 1) / RT_T, (E + RT_E - 1) / RT_E), dim3(256), 0, s, x,
                       W, T, D, E, gate_temp, fn, scores);
    return check_launch("router_tiled_kernel");
  }
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
