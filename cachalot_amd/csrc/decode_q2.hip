// Decode (one token) over a 2-bit affine g128 expert bank.
//
// Reference: src/cachalot/model/expert_affine.py:65-81 (rounding points),
// :117-152 (topk_core: experts summed in route order), moe_layer_metal.py:
// 93-130 (the traced block), mx.quantized_matmul's group formula
// s * sum(x q) + b * sum(x) (MLX qdot, as copied at minimax/codes_qmv.py:86-100).
//
//   q2_gate_up_kernel  one wave = R_GU rows of one expert.  Prologue per
//                      workgroup: (optionally) the top-k of the router scores,
//                      then the k slot lookups, into LDS.  Every weight,
//                      scale and bias load of the wave is issued before any
//                      arithmetic, with clamped addresses instead of branches,
//                      so a wave costs one memory round trip.  Lane l owns one
//                      64-code uint4 chunk per row (K = 4096: the whole row is
//                      one coalesced 1 KiB wave load per matrix).  Codes are
//                      spread into FP4 nibbles (code q in 0..3 is the E2M1
//                      encoding of q/2), converted to bf16 pairs by the gfx950
//                      converter with scale 2, and dotted with pre-paired bf16
//                      activations (v_dot2c_f32_bf16: exact products, fp32 sums).
//                      Epilogue: bf16(g), bf16(u), clamp,
//                      h = bf16(silu(g) * u * w_e), written in the pair order
//                      the down kernel consumes.
//   q2_down_kernel     one workgroup = RD rows of W2, k waves (wave e = expert
//                      e); lane l owns the 64-code chunk l of a row (one
//                      quantisation group: a 16-byte load, one scale, one bias;
//                      K = 2880 -> 45 chunks).  Each row value is rounded to
//                      bf16 (the reference's per-expert cast), handed over in
//                      LDS and summed in route order, + addend, -> fp32 / bf16.
#include "decode_common.h"
#include "router_launch.h"
#include "topk.h"

namespace cachalot {
namespace {

using namespace decode;
constexpr int R_GU = 4;     // rows per wave, gate/up
#ifndef Q2_DOWN_ROWS
#define Q2_DOWN_ROWS 8      // W2 rows per down workgroup
#endif

// Pair layout of a 16-value word: E_b = (v[4b], v[4b+2]), O_b = (v[4b+1], v[4b+3]);
// memory order E_0..E_3, O_0..O_3.  Position of value i (0..15) in uint16 units:
__device__ __forceinline__ int pair_pos(int i) {
  const int b = i >> 2, r = i & 3;
  return ((r & 1) ? 8 : 0) + 2 * b + (r >> 1);
}

// sum_i x_i * q_i over the 16 codes of word w, x pre-paired (xe = E pairs, xo = O pairs).
__device__ __forceinline__ float q2_word_dot(uint32_t w, const uint32_t* xe, const uint32_t* xo, float acc) {
  const uint32_t ev = w & 0x33333333u;
  const uint32_t od = (w >> 2) & 0x33333333u;
  acc = dot2_bf16(fp4x2_to_bf16x2<0>(ev, 2.0f), xe[0], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<0>(od, 2.0f), xo[0], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<1>(ev, 2.0f), xe[1], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<1>(od, 2.0f), xo[1], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<2>(ev, 2.0f), xe[2], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<2>(od, 2.0f), xo[2], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<3>(ev, 2.0f), xe[3], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<3>(od, 2.0f), xo[3], acc);
  return acc;
}

// (v0,v1),(v2,v3) -> E = (v0,v2), O = (v1,v3)
__device__ __forceinline__ void make_pairs(uint32_t a, uint32_t b, uint32_t& e, uint32_t& o) {
  e = (a & 0xffffu) | (b << 16);
  o = (a >> 16) | (b & 0xffff0000u);
}

constexpr uint32_t BF16_ONES = 0x3f803f80u;

// grid.x = ceil(k * ceil(F / R_GU) / WAVES); C = 64-code chunks per lane (D <= 4096 * C)
template <int C, bool FUSE>
__global__ void __launch_bounds__(64 * WAVES) q2_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L,
    const int32_t* __restrict__ slot_table, const int32_t* __restrict__ idx, const float* __restrict__ wts,
    RouteArgs ra, int D, int F, int E, int k, int group, float limit, uint16_t* __restrict__ hp,
    int32_t* __restrict__ ws_slots, float* __restrict__ ws_w) {
  __shared__ int s_slot[KMAX];
  __shared__ float s_w[KMAX];
  __shared__ int top_i[KMAX];
  __shared__ float top_v[KMAX];
  __shared__ float lds_v[16];
  __shared__ int lds_i[16];
  const int lane = threadIdx.x & 63;
  const int NC = D / 64;

  // activation chunk loads first: they do not depend on the routing
  uint4 xa[C][8];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = min(lane + 64 * i, NC - 1);
    const uint4* xp = reinterpret_cast<const uint4*>(x + (size_t)c * 64);
#pragma unroll
    for (int q = 0; q < 8; ++q) xa[i][q] = xp[q];
  }

  expert_prologue<FUSE>(slot_table, idx, wts, E, k, ra, s_slot, s_w, top_i, top_v, lds_v, lds_i, ws_slots, ws_w);

  const int RB = (F + R_GU - 1) / R_GU;
  const int item = blockIdx.x * WAVES + (threadIdx.x >> 6);
  if (item >= k * RB) return;
  const int e = item / RB;
  const int row0 = (item % RB) * R_GU;
  const int Fw = F / 16;
  uint16_t* hout = hp + (size_t)e * Fw * 16;
  const int slot = s_slot[e];
  if (slot < 0) {
    if (lane < R_GU && row0 + lane < F) hout[((row0 + lane) >> 4) * 16 + pair_pos((row0 + lane) & 15)] = 0;
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const int G = D / group;
  const uint4* w1 = reinterpret_cast<const uint4*>(base + L.off[0]);
  const uint16_t* s1 = reinterpret_cast<const uint16_t*>(base + L.off[1]);
  const uint16_t* b1 = reinterpret_cast<const uint16_t*>(base + L.off[2]);
  const uint4* w3 = reinterpret_cast<const uint4*>(base + L.off[6]);
  const uint16_t* s3 = reinterpret_cast<const uint16_t*>(base + L.off[7]);
  const uint16_t* b3 = reinterpret_cast<const uint16_t*>(base + L.off[8]);

  // every weight / scale / bias load of this wave, issued together
  uint4 vg[R_GU][C], vu[R_GU][C];
  uint16_t sg[R_GU][C], bg[R_GU][C], su[R_GU][C], bu[R_GU][C];
#pragma unroll
  for (int r = 0; r < R_GU; ++r) {
    const int n = min(row0 + r, F - 1);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int c = min(lane + 64 * i, NC - 1);
      const int g = (c * 64) / group;
      vg[r][i] = w1[(size_t)n * NC + c];
      vu[r][i] = w3[(size_t)n * NC + c];
      sg[r][i] = s1[(size_t)n * G + g];
      bg[r][i] = b1[(size_t)n * G + g];
      su[r][i] = s3[(size_t)n * G + g];
      bu[r][i] = b3[(size_t)n * G + g];
    }
  }
  // keep every load above this point in flight before any arithmetic
  __builtin_amdgcn_sched_barrier(0);

  // activation pairs and per-chunk sums
  uint32_t xe[C][4][4], xo[C][4][4];
  float xs[C];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const bool valid = lane + 64 * i < NC;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 a = xa[i][2 * j];
      const uint4 b = xa[i][2 * j + 1];
      make_pairs(a.x, a.y, xe[i][j][0], xo[i][j][0]);
      make_pairs(a.z, a.w, xe[i][j][1], xo[i][j][1]);
      make_pairs(b.x, b.y, xe[i][j][2], xo[i][j][2]);
      make_pairs(b.z, b.w, xe[i][j][3], xo[i][j][3]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (!valid) xe[i][j][q] = xo[i][j][q] = 0u;
        sum = dot2_bf16(xe[i][j][q], BF16_ONES, sum);
        sum = dot2_bf16(xo[i][j][q], BF16_ONES, sum);
      }
    }
    xs[i] = sum;
  }

  float part[2 * R_GU];
#pragma unroll
  for (int r = 0; r < R_GU; ++r) {
    float pg = 0.0f, pu = 0.0f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      float dg = 0.0f, du = 0.0f;
      dg = q2_word_dot(vg[r][i].x, xe[i][0], xo[i][0], dg);
      du = q2_word_dot(vu[r][i].x, xe[i][0], xo[i][0], du);
      dg = q2_word_dot(vg[r][i].y, xe[i][1], xo[i][1], dg);
      du = q2_word_dot(vu[r][i].y, xe[i][1], xo[i][1], du);
      dg = q2_word_dot(vg[r][i].z, xe[i][2], xo[i][2], dg);
      du = q2_word_dot(vu[r][i].z, xe[i][2], xo[i][2], du);
      dg = q2_word_dot(vg[r][i].w, xe[i][3], xo[i][3], dg);
      du = q2_word_dot(vu[r][i].w, xe[i][3], xo[i][3], du);
      pg = pg + (bf16_to_f32(sg[r][i]) * dg + bf16_to_f32(bg[r][i]) * xs[i]);
      pu = pu + (bf16_to_f32(su[r][i]) * du + bf16_to_f32(bu[r][i]) * xs[i]);
    }
    part[2 * r] = pg;
    part[2 * r + 1] = pu;
  }
  // value 2r+v ends in lanes [8(2r+v), 8(2r+v)+8)
  const float red = wave_transpose_sum<2 * R_GU>(part, lane);
  const float up = __shfl(red, lane + 8, 64);
  if ((lane & 15) == 0) {
    const int n = row0 + (lane >> 4);
    if (n < F) {
      float g = round_bf16(red);
      float u = round_bf16(up);
      if (limit > 0.0f) {
        u = fminf(fmaxf(u, -limit), limit);
        g = fminf(g, limit);
      }
      const float h = (silu_f32(g) * u) * s_w[e];
      hout[(n >> 4) * 16 + pair_pos(n & 15)] = f32_to_bf16(h);
    }
  }
}

// grid.x = ceil(D / RD); one workgroup = k waves, wave e = expert e, RD rows.
// Lane l owns the 64-code chunk l of a row (words 4l .. 4l+3, one quantisation
// group): one 16-byte weight load, one scale and one bias per row; lanes past
// the row's last chunk (K = 2880: 45 chunks) only take part in the reductions.
// The expert's hidden pairs for the lane's chunk are loaded once and reused for
// all RD rows.
template <int RD>
__global__ void __launch_bounds__(64 * KMAX) q2_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, const int32_t* __restrict__ ws_slots, int D, int F, int k,
    int group, const uint16_t* __restrict__ hp, const uint16_t* __restrict__ addend, float* __restrict__ routed,
    uint16_t* __restrict__ out) {
  __shared__ float vals[KMAX][RD];
  const int lane = threadIdx.x & 63;
  const int e = threadIdx.x >> 6;
  const int row0 = blockIdx.x * RD;
  const int Kw = F / 16;                   // valid words per row
  const int NCH = (Kw + 3) / 4;            // 64-code chunks per row (the last may be partial)
  const int G = (F + group - 1) / group;   // groups per row (the last may be partial)
  const int stride = G * group / 16;       // stored words per row
  const int c = min(lane, NCH - 1);
  const bool active = lane < NCH;
  const int g = (c * 64) / group;
  const int slot = ws_slots[e];

  float rowv[RD];
#pragma unroll
  for (int r = 0; r < RD; ++r) rowv[r] = 0.0f;
  if (slot >= 0) {
    const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(base + L.off[3]);
    const uint16_t* s2 = reinterpret_cast<const uint16_t*>(base + L.off[4]);
    const uint16_t* b2 = reinterpret_cast<const uint16_t*>(base + L.off[5]);
    const uint4* hpe = reinterpret_cast<const uint4*>(hp + (size_t)e * Kw * 16);
    uint4 hv[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = min(4 * c + q, Kw - 1);
      hv[2 * q] = hpe[2 * j];
      hv[2 * q + 1] = hpe[2 * j + 1];
    }
    uint4 wv[RD];
    uint16_t sv[RD], bv[RD];
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      const int n = min(row0 + r, D - 1);
      // the chunk's words: 4 whole words unless the row ends inside it (then the
      // missing words are padding codes, multiplied by zeroed hidden pairs below)
      wv[r] = *reinterpret_cast<const uint4*>(w2 + (size_t)n * stride + 4 * c);
      sv[r] = s2[(size_t)n * G + g];
      bv[r] = b2[(size_t)n * G + g];
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t he[4][4], ho[4][4];
    float hs = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool valid = active && (4 * c + q < Kw);
      he[q][0] = valid ? hv[2 * q].x : 0u; he[q][1] = valid ? hv[2 * q].y : 0u;
      he[q][2] = valid ? hv[2 * q].z : 0u; he[q][3] = valid ? hv[2 * q].w : 0u;
      ho[q][0] = valid ? hv[2 * q + 1].x : 0u; ho[q][1] = valid ? hv[2 * q + 1].y : 0u;
      ho[q][2] = valid ? hv[2 * q + 1].z : 0u; ho[q][3] = valid ? hv[2 * q + 1].w : 0u;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        hs = dot2_bf16(he[q][p], BF16_ONES, hs);
        hs = dot2_bf16(ho[q][p], BF16_ONES, hs);
      }
    }
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      float d = 0.0f;
      d = q2_word_dot(wv[r].x, he[0], ho[0], d);
      d = q2_word_dot(wv[r].y, he[1], ho[1], d);
      d = q2_word_dot(wv[r].z, he[2], ho[2], d);
      d = q2_word_dot(wv[r].w, he[3], ho[3], d);
      rowv[r] = bf16_to_f32(sv[r]) * d + bf16_to_f32(bv[r]) * hs;
    }
  }
  // row sums (row r ends in lanes [r * 64/RD, (r+1) * 64/RD)); the wave hands its
  // expert's bf16-rounded rows to LDS
  const float red = wave_transpose_sum<RD>(rowv, lane);
  if ((lane & (64 / RD - 1)) == 0) vals[e][lane / (64 / RD)] = round_bf16(red);
  __syncthreads();
  const int t = threadIdx.x;
  if (t < RD && row0 + t < D) {
    const int n = row0 + t;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) acc = acc + vals[j][t];
    if (routed) routed[n] = acc;
    if (out) out[n] = f32_to_bf16(addend ? acc + bf16_to_f32(addend[n]) : acc);
  }
}

}  // namespace

size_t q2_workspace_bytes(int D, int F, int k) {
  (void)D;
  return ws_offsets((size_t)k * ((F + 15) / 16) * 16 * sizeof(uint16_t)).total;
}

int launch_q2_decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                     const int32_t* slot_table, const int32_t* idx, const float* w, const RouteArgs* ra, int D,
                     int F, int E, int k, int group, float swiglu_limit, const uint16_t* addend, float* routed,
                     uint16_t* out, void* workspace, size_t workspace_bytes, hipStream_t s) {
  CACHALOT_REQUIRE(pool && layout && slot_table && x, "moe_decode_q2: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_q2: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_q2: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(E >= 1 && E <= 1024, "moe_decode_q2: E=%d outside 1..1024", E);
  CACHALOT_REQUIRE(group == 64 || group == 128, "moe_decode_q2: group_size %d (64 or 128)", group);
  CACHALOT_REQUIRE(D % group == 0 && D >= 64 && D <= 8192,
                   "moe_decode_q2: D=%d must be a multiple of group %d and <= 8192", D, group);
  CACHALOT_REQUIRE(F % 16 == 0 && F >= 64 && F <= 4096, "moe_decode_q2: F=%d must be a multiple of 16 in 64..4096",
                   F);
  const WsOffsets wo = ws_offsets((size_t)k * ((F + 15) / 16) * 16 * sizeof(uint16_t));
  if (workspace == nullptr || workspace_bytes < wo.total)
    return fail(CACHALOT_ESPACE, "moe_decode_q2: workspace %zu < %zu bytes", workspace_bytes, wo.total);
  Layout L;
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  int rc = make_layout(layout, 9, used, L, "moe_decode_q2");
  if (rc) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* hp = reinterpret_cast<uint16_t*>(ws + wo.hidden);
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
      hipLaunchKernelGGL((q2_gate_up_kernel<1, true>), dim3(blocks), dim3(64 * WAVES), lds, s, x, pool, L, slot_table,
                         idx, w, r, D, F, E, k, group, swiglu_limit, hp, ws_slots, ws_w);
    else
      hipLaunchKernelGGL((q2_gate_up_kernel<2, true>), dim3(blocks), dim3(64 * WAVES), lds, s, x, pool, L, slot_table,
                         idx, w, r, D, F, E, k, group, swiglu_limit, hp, ws_slots, ws_w);
  } else {
    if (c1)
      hipLaunchKernelGGL((q2_gate_up_kernel<1, false>), dim3(blocks), dim3(64 * WAVES), 0, s, x, pool, L, slot_table,
                         idx, w, r, D, F, E, k, group, swiglu_limit, hp, ws_slots, ws_w);
    else
      hipLaunchKernelGGL((q2_gate_up_kernel<2, false>), dim3(blocks), dim3(64 * WAVES), 0, s, x, pool, L, slot_table,
                         idx, w, r, D, F, E, k, group, swiglu_limit, hp, ws_slots, ws_w);
  }
  rc = check_launch("q2_gate_up_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((q2_down_kernel<Q2_DOWN_ROWS>), dim3((D + Q2_DOWN_ROWS - 1) / Q2_DOWN_ROWS), dim3(64 * k), 0, s,
                     pool, L, ws_slots, D, F, k, group, hp, addend, routed, out);
  return check_launch("q2_down_kernel");
}

}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_q2_workspace_bytes(int D, int F, int k) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX) return 0;
  return cachalot::q2_workspace_bytes(D, F, k);
}

extern "C" int cachalot_moe_decode_q2(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                                      const int32_t* slot_table, const int32_t* idx, const float* w, int D, int F,
                                      int E, int k, int group, float swiglu_limit, const uint16_t* addend,
                                      float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                      cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(idx && w, "moe_decode_q2: null pointer");
  return launch_q2_decode(x, pool, layout, slot_table, idx, w, nullptr, D, F, E, k, group, swiglu_limit, addend,
                          routed, out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cachalot_moe_layer_decode_q2(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                            int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                            int order, const uint8_t* pool, const cachalot_expert_layout* layout,
                                            const int32_t* slot_table, int D, int F, int group, float swiglu_limit,
                                            const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                            float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                            cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_q2: null router pointer");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_q2: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_q2: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_q2: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_q2: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_q2: invalid topk=%d for %d experts", k, E);
  hipStream_t s = (hipStream_t)stream;
  int rc = launch_router_scores(x, gate_weight, 1, D, E, gate_temp, score_fn, scores, s);
  if (rc) return rc;
  RouteArgs ra{scores, gate_bias, E, order, norm, route_scale, idx_out, w_out};
  return launch_q2_decode(x, pool, layout, slot_table, nullptr, nullptr, &ra, D, F, E, k, group, swiglu_limit,
                          addend, routed, out, workspace, workspace_bytes, s);
}
