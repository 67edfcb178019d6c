// Decode (one token) over an FP4 E2M1 / E8M0-block-32 expert bank.
//
// Reference: src/cachalot/model/moe_fused_metal.py:189-233 (fused_gate_up +
// fused_down): x read as fp32, gate/up accumulated in fp32,
// h = silu(min(g, L)) * clip(u, -L, L) * w_e in fp32 (:127-135), out = sum_e
// W2_e h_e in fp32 with experts in route order (:160-178).  No bf16 rounding
// point anywhere on this path.
//
//   fp4_gate_up_kernel  one wave = R rows of one expert (same prologue and
//                       load-everything-first structure as the 2-bit kernel);
//                       lane l owns 64 codes (two E8M0 blocks, 32 bytes) of the
//                       row, so K = 4096 is a 2 KiB coalesced wave load per
//                       matrix.  Nibbles become bf16 pairs (value * 2^e, exact)
//                       in the gfx950 converter and meet the bf16 activation
//                       pairs in v_dot2c_f32_bf16.
//   fp4_down_kernel     one workgroup = R rows of W2, k waves (wave e = expert
//                       e); lane l owns words l + 64 i of the row (8 codes each);
//                       the fp32 hidden vector stays fp32 (converter to f32
//                       pairs, fp32 FMA); per-expert row values meet in LDS and
//                       are summed in route order.
#include "decode_common.h"
#include "router_launch.h"

namespace cachalot {
namespace {

using namespace decode;
constexpr int R_GU = 4;
constexpr int MAXW = 6;   // 8-code words per lane, down (F <= 3072)

__device__ __forceinline__ float fp4_word_dot_bf16(uint32_t w, float scale, const uint32_t* xp, float acc) {
  acc = dot2_bf16(fp4x2_to_bf16x2<0>(w, scale), xp[0], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<1>(w, scale), xp[1], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<2>(w, scale), xp[2], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<3>(w, scale), xp[3], acc);
  return acc;
}

// 8 uint32 words of one 64-code chunk (two scale blocks) dotted with 32 bf16 pairs of x.
__device__ __forceinline__ float fp4_chunk_dot(uint4 a, uint4 b, float s0, float s1, const uint32_t* xw) {
  float acc = 0.0f;
  acc = fp4_word_dot_bf16(a.x, s0, xw + 0, acc);
  acc = fp4_word_dot_bf16(a.y, s0, xw + 4, acc);
  acc = fp4_word_dot_bf16(a.z, s0, xw + 8, acc);
  acc = fp4_word_dot_bf16(a.w, s0, xw + 12, acc);
  acc = fp4_word_dot_bf16(b.x, s1, xw + 16, acc);
  acc = fp4_word_dot_bf16(b.y, s1, xw + 20, acc);
  acc = fp4_word_dot_bf16(b.z, s1, xw + 24, acc);
  acc = fp4_word_dot_bf16(b.w, s1, xw + 28, acc);
  return acc;
}

template <int C, bool FUSE>
__global__ void __launch_bounds__(64 * WAVES) fp4_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L,
    const int32_t* __restrict__ slot_table, const int32_t* __restrict__ idx, const float* __restrict__ wts,
    RouteArgs ra, int D, int F, int E, int k, float limit, float* __restrict__ hidden,
    int32_t* __restrict__ ws_slots, float* __restrict__ ws_w) {
  __shared__ int s_slot[KMAX];
  __shared__ float s_w[KMAX];
  __shared__ int top_i[KMAX];
  __shared__ float top_v[KMAX];
  __shared__ float lds_v[16];
  __shared__ int lds_i[16];
  const int lane = threadIdx.x & 63;
  const int NC = D / 64;
  const int SB = D / 32;

  uint32_t xw[C][32];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = min(lane + 64 * i, NC - 1);
    const uint4* xp = reinterpret_cast<const uint4*>(x + (size_t)c * 64);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 v = xp[q];
      xw[i][4 * q] = v.x; xw[i][4 * q + 1] = v.y; xw[i][4 * q + 2] = v.z; xw[i][4 * q + 3] = v.w;
    }
  }

  expert_prologue<FUSE>(slot_table, idx, wts, E, k, ra, s_slot, s_w, top_i, top_v, lds_v, lds_i, ws_slots, ws_w);

  const int RB = (F + R_GU - 1) / R_GU;
  const int item = blockIdx.x * WAVES + (threadIdx.x >> 6);
  if (item >= k * RB) return;
  const int e = item / RB;
  const int row0 = (item % RB) * R_GU;
  float* hout = hidden + (size_t)e * F;
  const int slot = s_slot[e];
  if (slot < 0) {
    if (lane < R_GU && row0 + lane < F) hout[row0 + lane] = 0.0f;
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const uint4* w1 = reinterpret_cast<const uint4*>(base + L.off[0]);
  const uint8_t* s1 = base + L.off[1];
  const uint4* w3 = reinterpret_cast<const uint4*>(base + L.off[6]);
  const uint8_t* s3 = base + L.off[7];

  uint4 ga[R_GU][C], gb[R_GU][C], ua[R_GU][C], ub[R_GU][C];
  uint8_t sg0[R_GU][C], sg1[R_GU][C], su0[R_GU][C], su1[R_GU][C];
#pragma unroll
  for (int r = 0; r < R_GU; ++r) {
    const int n = min(row0 + r, F - 1);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int c = min(lane + 64 * i, NC - 1);
      ga[r][i] = w1[((size_t)n * NC + c) * 2];
      gb[r][i] = w1[((size_t)n * NC + c) * 2 + 1];
      ua[r][i] = w3[((size_t)n * NC + c) * 2];
      ub[r][i] = w3[((size_t)n * NC + c) * 2 + 1];
      sg0[r][i] = s1[(size_t)n * SB + 2 * c];
      sg1[r][i] = s1[(size_t)n * SB + 2 * c + 1];
      su0[r][i] = s3[(size_t)n * SB + 2 * c];
      su1[r][i] = s3[(size_t)n * SB + 2 * c + 1];
    }
  }
  // keep every load above this point in flight before any arithmetic
  __builtin_amdgcn_sched_barrier(0);

  float part[2 * R_GU];
#pragma unroll
  for (int r = 0; r < R_GU; ++r) {
    float pg = 0.0f, pu = 0.0f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float valid = (lane + 64 * i < NC) ? 1.0f : 0.0f;
      pg = pg + valid * fp4_chunk_dot(ga[r][i], gb[r][i], e8m0_to_f32(sg0[r][i]), e8m0_to_f32(sg1[r][i]), xw[i]);
      pu = pu + valid * fp4_chunk_dot(ua[r][i], ub[r][i], e8m0_to_f32(su0[r][i]), e8m0_to_f32(su1[r][i]), xw[i]);
    }
    part[2 * r] = pg;
    part[2 * r + 1] = pu;
  }
  const float red = wave_transpose_sum<2 * R_GU>(part, lane);
  const float up = __shfl(red, lane + 8, 64);
  if ((lane & 15) == 0) {
    const int n = row0 + (lane >> 4);
    if (n < F) {
      float g = red, u = up;
      if (limit > 0.0f) {
        u = fminf(fmaxf(u, -limit), limit);
        g = fminf(g, limit);
      }
      hout[n] = (silu_f32(g) * u) * s_w[e];
    }
  }
}

// grid.x = ceil(D / R_DN); one workgroup = k waves, wave e = expert e
__global__ void __launch_bounds__(64 * KMAX) fp4_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, const int32_t* __restrict__ ws_slots, int D, int F, int k,
    const float* __restrict__ hidden, const uint16_t* __restrict__ addend, float* __restrict__ routed,
    uint16_t* __restrict__ out) {
  __shared__ float vals[KMAX][R_DN];
  const int lane = threadIdx.x & 63;
  const int e = threadIdx.x >> 6;
  const int row0 = blockIdx.x * R_DN;
  const int Kw = F / 8;     // 32-bit words per row
  const int SB = F / 32;    // scale blocks per row
  const int slot = ws_slots[e];
  float rowv[R_DN];
#pragma unroll
  for (int r = 0; r < R_DN; ++r) rowv[r] = 0.0f;
  if (slot >= 0) {
    const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(base + L.off[3]);
    const uint8_t* s2 = base + L.off[4];
    const float4* he = reinterpret_cast<const float4*>(hidden + (size_t)e * F);
    uint32_t wv[R_DN][MAXW];
    uint8_t sv[R_DN][MAXW];
    float4 ha[MAXW], hb[MAXW];
#pragma unroll
    for (int i = 0; i < MAXW; ++i) {
      const int j = min(lane + 64 * i, Kw - 1);
      ha[i] = he[2 * j];
      hb[i] = he[2 * j + 1];
    }
#pragma unroll
    for (int r = 0; r < R_DN; ++r) {
      const int n = min(row0 + r, D - 1);
#pragma unroll
      for (int i = 0; i < MAXW; ++i) {
        const int j = min(lane + 64 * i, Kw - 1);
        wv[r][i] = w2[(size_t)n * Kw + j];
        sv[r][i] = s2[(size_t)n * SB + (j >> 2)];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R_DN; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < MAXW; ++i) {
        const float valid = (lane + 64 * i < Kw) ? 1.0f : 0.0f;
        const float sc = e8m0_to_f32(sv[r][i]);
        const float2_t p0 = fp4x2_to_f32x2<0>(wv[r][i], sc);
        const float2_t p1 = fp4x2_to_f32x2<1>(wv[r][i], sc);
        const float2_t p2 = fp4x2_to_f32x2<2>(wv[r][i], sc);
        const float2_t p3 = fp4x2_to_f32x2<3>(wv[r][i], sc);
        float d = 0.0f;
        d = __builtin_fmaf(p0[0], ha[i].x, d);
        d = __builtin_fmaf(p0[1], ha[i].y, d);
        d = __builtin_fmaf(p1[0], ha[i].z, d);
        d = __builtin_fmaf(p1[1], ha[i].w, d);
        d = __builtin_fmaf(p2[0], hb[i].x, d);
        d = __builtin_fmaf(p2[1], hb[i].y, d);
        d = __builtin_fmaf(p3[0], hb[i].z, d);
        d = __builtin_fmaf(p3[1], hb[i].w, d);
        acc = __builtin_fmaf(valid, d, acc);
      }
      rowv[r] = acc;
    }
  }
  const float red = wave_transpose_sum<R_DN>(rowv, lane);
  combine_rows<false>(red, lane, e, row0, D, k, vals, addend, routed, out);
}

}  // namespace

size_t fp4_workspace_bytes(int D, int F, int k) {
  (void)D;
  return ws_offsets((size_t)k * F * sizeof(float)).total;
}

int launch_fp4_decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                      const int32_t* slot_table, const int32_t* idx, const float* w, const RouteArgs* ra, int D,
                      int F, int E, int k, float swiglu_limit, const uint16_t* addend, float* routed, uint16_t* out,
                      void* workspace, size_t workspace_bytes, hipStream_t s) {
  CACHALOT_REQUIRE(pool && layout && slot_table && x, "moe_decode_fp4: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_fp4: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_fp4: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(E >= 1 && E <= 1024, "moe_decode_fp4: E=%d outside 1..1024", E);
  CACHALOT_REQUIRE(D % 64 == 0 && D >= 64 && D <= 8192, "moe_decode_fp4: D=%d must be a multiple of 64 and <= 8192",
                   D);
  CACHALOT_REQUIRE(F % 32 == 0 && F >= 32 && F <= 8 * 64 * MAXW,
                   "moe_decode_fp4: F=%d must be a multiple of 32 and <= %d", F, 8 * 64 * MAXW);
  const WsOffsets wo = ws_offsets((size_t)k * F * sizeof(float));
  if (workspace == nullptr || workspace_bytes < wo.total)
    return fail(CACHALOT_ESPACE, "moe_decode_fp4: workspace %zu < %zu bytes", workspace_bytes, wo.total);
  Layout L;
  static const int used[6] = {0, 1, 3, 4, 6, 7};
  int rc = make_layout(layout, 6, used, L, "moe_decode_fp4");
  if (rc) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* hidden = reinterpret_cast<float*>(ws + wo.hidden);
  int32_t* ws_slots = reinterpret_cast<int32_t*>(ws + wo.slots);
  float* ws_w = reinterpret_cast<float*>(ws + wo.weights);
  RouteArgs none{};
  const RouteArgs& r = ra ? *ra : none;
  const int items = k * ((F + R_GU - 1) / R_GU);
  const int blocks = (items + WAVES - 1) / WAVES;
  const size_t lds = 0;
  const bool c1 = D <= 4096;
  if (ra) {
    if (c1)
      hipLaunchKernelGGL((fp4_gate_up_kernel<1, true>), dim3(blocks), dim3(64 * WAVES), lds, s, x, pool, L,
                         slot_table, idx, w, r, D, F, E, k, swiglu_limit, hidden, ws_slots, ws_w);
    else
      hipLaunchKernelGGL((fp4_gate_up_kernel<2, true>), dim3(blocks), dim3(64 * WAVES), lds, s, x, pool, L,
                         slot_table, idx, w, r, D, F, E, k, swiglu_limit, hidden, ws_slots, ws_w);
  } else {
    if (c1)
      hipLaunchKernelGGL((fp4_gate_up_kernel<1, false>), dim3(blocks), dim3(64 * WAVES), 0, s, x, pool, L,
                         slot_table, idx, w, r, D, F, E, k, swiglu_limit, hidden, ws_slots, ws_w);
    else
      hipLaunchKernelGGL((fp4_gate_up_kernel<2, false>), dim3(blocks), dim3(64 * WAVES), 0, s, x, pool, L,
                         slot_table, idx, w, r, D, F, E, k, swiglu_limit, hidden, ws_slots, ws_w);
  }
  rc = check_launch("fp4_gate_up_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(fp4_down_kernel, dim3((D + R_DN - 1) / R_DN), dim3(64 * k), 0, s, pool, L, ws_slots, D, F, k,
                     hidden, addend, routed, out);
  return check_launch("fp4_down_kernel");
}

}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_fp4_workspace_bytes(int D, int F, int k) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX) return 0;
  return cachalot::fp4_workspace_bytes(D, F, k);
}

extern "C" int cachalot_moe_decode_fp4(const uint16_t* x, const uint8_t* pool,
                                       const cachalot_expert_layout* layout, const int32_t* slot_table,
                                       const int32_t* idx, const float* w, int D, int F, int E, int k,
                                       float swiglu_limit, const uint16_t* addend, float* routed, uint16_t* out,
                                       void* workspace, size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(idx && w, "moe_decode_fp4: null pointer");
  return launch_fp4_decode(x, pool, layout, slot_table, idx, w, nullptr, D, F, E, k, swiglu_limit, addend, routed,
                           out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cachalot_moe_layer_decode_fp4(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                             int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                             int order, const uint8_t* pool, const cachalot_expert_layout* layout,
                                             const int32_t* slot_table, int D, int F, float swiglu_limit,
                                             const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                             float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                             cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_fp4: null router pointer");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_fp4: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_fp4: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_fp4: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_fp4: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_fp4: invalid topk=%d for %d experts", k, E);
  hipStream_t s = (hipStream_t)stream;
  int rc = launch_router_scores(x, gate_weight, 1, D, E, gate_temp, score_fn, scores, s);
  if (rc) return rc;
  RouteArgs ra{scores, gate_bias, E, order, norm, route_scale, idx_out, w_out};
  return launch_fp4_decode(x, pool, layout, slot_table, nullptr, nullptr, &ra, D, F, E, k, swiglu_limit, addend,
                           routed, out, workspace, workspace_bytes, s);
}
