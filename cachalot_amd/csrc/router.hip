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
  if ((int)threadIdx.x < tail.k) {
    tail.ws_slots[threadIdx.x] = top_s[threadIdx.x];
    tail.ws_w[threadIdx.x] = w[threadIdx.x];
    if (tail.idx_out) tail.idx_out[threadIdx.x] = top_i[threadIdx.x];
    if (tail.w_out) tail.w_out[threadIdx.x] = w[threadIdx.x];
  }
  if (threadIdx.x == 0) __hip_atomic_store(tail.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave per expert row (lane l owns chunk l of D/64 elements), TT tokens per
// wave, blockDim / 64 waves per workgroup; optionally the top-k tail (one token).
template <int TT, int NV>
__global__ void __launch_bounds__(256) router_scores_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ W, int T, int D,
                                                            int E, float gate_temp, int fn,
                                                            float* __restrict__ scores, decode::RouteTail tail,
                                                            uint8_t* __restrict__ xplanes) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (xplanes != nullptr && blockIdx.y == 0) {   // token 0 as fp8 planes for the matrix-core decode
    for (int t4 = blockIdx.x * blockDim.x + threadIdx.x; 4 * t4 < D; t4 += gridDim.x * blockDim.x)
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

// Many tokens: one 256-thread workgroup = 64 tokens x 32 experts, each thread 4
// tokens (tq + 16 a) x 2 experts (eq + 16 b).  The same arithmetic as router_row:
// chunk c (of 64) of every dot product is a sequential fp32 sum of its D/64
// products in k order, and the 64 chunk sums meet in the pairwise tree (left +
// right) the xor butterfly forms, kept as a binary-counter stack of six partial
// nodes per dot product.  Chunk by chunk, the x and W slices are staged in LDS as
// bf16 (double-buffered, one barrier per chunk) and read as 8-value runs (one
// 16-byte read per token or expert feeds 8 x 4 products); rows are padded to an
// odd number of 16-byte slots so the 16 experts a wave row reads hit distinct
// bank groups.  fma(x, w, s) equals s + x * w here: the product of two bf16
// values is exact in fp32 (16 significant bits) unless it is below 2^-133.
constexpr int RT_TA = 4;             // tokens per thread (tq + 16 a)
constexpr int RT_TB = 2;             // experts per thread (eq + 16 b)
constexpr int RT_T = 16 * RT_TA;     // tokens per workgroup
constexpr int RT_E = 16 * RT_TB;     // experts per workgroup
constexpr int RT_MAXCH = 80;         // D / 64 <= 80 (D <= 5120)
constexpr int RT_MAXS = RT_MAXCH * 2 + 32;   // staged row bytes, padding included
constexpr int RT_MIN_T = 1024;       // fewer tokens: the 4-token kernel fills the chip better

__host__ __device__ inline int rt_stride(int ch) { return ch * 2 + ((ch / 8) % 2 == 0 ? 16 : 32); }

// Chunk c of a tile's x rows, then its W rows, as 16-byte items (rows past T / E:
// clamped, unused), and the store of those items into a staged buffer.
template <int N>
__device__ __forceinline__ void rt_load(uint4 (&v)[N], const uint16_t* __restrict__ x, const uint16_t* __restrict__ W,
                                        int T, int D, int E, int t0, int e0, int c, int tid, int items, int per_row) {
  const int ch = 8 * per_row;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int it = min(tid + 256 * j, items - 1);
    const int r = it / per_row, q = it - r * per_row;
    const uint16_t* src = r < RT_T ? x + (size_t)min(t0 + r, T - 1) * D : W + (size_t)min(e0 + r - RT_T, E - 1) * D;
    v[j] = *reinterpret_cast<const uint4*>(src + c * ch + 8 * q);
  }
}

template <int N>
__device__ __forceinline__ void rt_store(uint8_t* buf, const uint4 (&v)[N], int tid, int items, int per_row, int S) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int it = tid + 256 * j;
    const int r = it / per_row, q = it - r * per_row;
    if (it < items) *reinterpret_cast<uint4*>(buf + r * S + 16 * q) = v[j];
  }
}

__global__ void __launch_bounds__(256) router_tiled_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ W, int T, int D, int E,
                                                           float gate_temp, int fn, float* __restrict__ scores) {
  __shared__ __align__(16) uint8_t st[2][(RT_T + RT_E) * RT_MAXS];
  const int tid = threadIdx.x;
  const int eq = tid & 15, tq = tid >> 4;
  const int t0 = blockIdx.x * RT_T, e0 = blockIdx.y * RT_E;
  const int per_row = D / 512;                // 16-byte items per staged row
  const int ch = 8 * per_row;                 // D / 64
  const int S = rt_stride(ch);
  const int items = (RT_T + RT_E) * per_row;  // x rows first, then W rows
  constexpr int MAXIT = ((RT_T + RT_E) * RT_MAXCH / 8 + 255) / 256;

  float stk[6][RT_TA * RT_TB];
  float node[RT_TA * RT_TB];
  uint4 v[MAXIT];
  rt_load(v, x, W, T, D, E, t0, e0, 0, tid, items, per_row);
  rt_store(st[0], v, tid, items, per_row, S);
  __syncthreads();
  for (int c = 0; c < CHUNKS; ++c) {
    if (c + 1 < CHUNKS) rt_load(v, x, W, T, D, E, t0, e0, c + 1, tid, items, per_row);
    const uint8_t* buf = st[c & 1];
    float acc[RT_TA * RT_TB];
#pragma unroll
    for (int p = 0; p < RT_TA * RT_TB; ++p) acc[p] = 0.0f;
    // (a runtime loop: unrolled, the scheduled-ahead reads push the kernel to one wave per SIMD)
    for (int k8 = 0; k8 < per_row; ++k8) {
      uint4 xa[RT_TA], wb[RT_TB];
#pragma unroll
      for (int a = 0; a < RT_TA; ++a) xa[a] = *reinterpret_cast<const uint4*>(buf + (tq + 16 * a) * S + 16 * k8);
#pragma unroll
      for (int b = 0; b < RT_TB; ++b)
        wb[b] = *reinterpret_cast<const uint4*>(buf + (RT_T + eq + 16 * b) * S + 16 * k8);
#pragma unroll
      for (int h = 0; h < 4; ++h) {            // the 8 values in k order: word h, low then high half
        float xl[RT_TA], xh[RT_TA], wl[RT_TB], wh[RT_TB];
#pragma unroll
        for (int a = 0; a < RT_TA; ++a) {
          const uint32_t u = h == 0 ? xa[a].x : h == 1 ? xa[a].y : h == 2 ? xa[a].z : xa[a].w;
          xl[a] = __uint_as_float(u << 16);
          xh[a] = __uint_as_float(u & 0xffff0000u);
        }
#pragma unroll
        for (int b = 0; b < RT_TB; ++b) {
          const uint32_t u = h == 0 ? wb[b].x : h == 1 ? wb[b].y : h == 2 ? wb[b].z : wb[b].w;
          wl[b] = __uint_as_float(u << 16);
          wh[b] = __uint_as_float(u & 0xffff0000u);
        }
#pragma unroll
        for (int a = 0; a < RT_TA; ++a)
#pragma unroll
          for (int b = 0; b < RT_TB; ++b) {
            float t = acc[RT_TB * a + b];
            t = __builtin_fmaf(xl[a], wl[b], t);
            t = __builtin_fmaf(xh[a], wh[b], t);
            acc[RT_TB * a + b] = t;
          }
      }
    }
    if (c + 1 < CHUNKS) rt_store(st[(c + 1) & 1], v, tid, items, per_row, S);
    // merge chunk c into the tree (c is uniform: every branch below is too)
#pragma unroll
    for (int p = 0; p < RT_TA * RT_TB; ++p) node[p] = acc[p];
    // chunk c closes the nodes of the levels below its lowest zero bit
    const int up = __builtin_ctz(~c);   // levels merged (6 after the last chunk)
#pragma unroll
    for (int L = 0; L < 6; ++L) {
      if (L < up) {
#pragma unroll
        for (int p = 0; p < RT_TA * RT_TB; ++p) node[p] = stk[L][p] + node[p];
      } else if (L == up) {
#pragma unroll
        for (int p = 0; p < RT_TA * RT_TB; ++p) stk[L][p] = node[p];
      }
    }
    __syncthreads();
  }
  // after chunk 63 every level merged: node holds the root
#pragma unroll
  for (int a = 0; a < RT_TA; ++a) {
    const int t = t0 + tq + 16 * a;
    if (t >= T) continue;
#pragma unroll
    for (int b = 0; b < RT_TB; ++b) {
      const int e = e0 + eq + 16 * b;
      if (e < E) scores[(size_t)t * E + e] = score_of(node[RT_TB * a + b] / gate_temp, fn);
    }
  }
}

}  // namespace

template <int TT>
static void launch_scores_tt(const uint16_t* x, const uint16_t* W, int T, int D, int E, float temp, int fn,
                             float* scores, hipStream_t s, const decode::RouteTail& tail, uint8_t* xplanes) {
  // one token: one wave per workgroup, so the E rows spread over every CU
  const int wpb = TT == 1 ? 1 : 4;
  const dim3 grid((E + wpb - 1) / wpb, (T + TT - 1) / TT), block(64 * wpb);
  switch (D) {
    case 4096: hipLaunchKernelGGL((router_scores_kernel<TT, 8>), grid, block, 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    case 5120: hipLaunchKernelGGL((router_scores_kernel<TT, 10>), grid, block, 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    case 7168: hipLaunchKernelGGL((router_scores_kernel<TT, 14>), grid, block, 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
    default: hipLaunchKernelGGL((router_scores_kernel<TT, 0>), grid, block, 0, s, x, W, T, D, E, temp, fn, scores, tail, xplanes); break;
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
  // tokens per wave: 4 from 8 tokens on, 2 below (twice the waves for a small batch:
  // B = 4 68.4 against 70 us per batched step; at B = 32, 2 per wave lost 2.6 us)
  if (T >= 8) launch_scores_tt<4>(x, W, T, D, E, gate_temp, fn, scores, s, none, nullptr);
  else if (T >= 4) launch_scores_tt<2>(x, W, T, D, E, gate_temp, fn, scores, s, none, nullptr);
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
