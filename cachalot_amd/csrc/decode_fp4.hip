// Decode (one token) over an FP4 E2M1 / E8M0-block-32 expert bank.
//
// Reference: src/cachalot/model/moe_fused_metal.py:189-233 (fused_gate_up +
// fused_down): x read as fp32, gate/up accumulated in fp32,
// h = silu(min(g, L)) * clip(u, -L, L) * w_e in fp32 (:127-135), out = sum_e
// W2_e h_e in fp32 with experts in route order (:160-178).  No bf16 rounding
// point anywhere on this path.
//
//   fp4_gate_up_kernel  one wave = R rows of one expert; lane l owns 64 codes
//                       (two E8M0 blocks, 32 bytes) of the row, so K = 4096 is a
//                       2 KiB coalesced wave load per matrix.  Nibbles become
//                       bf16 pairs (value * 2^e, exact) in the gfx950 converter
//                       and meet the bf16 activation pairs in v_dot2c_f32_bf16.
//   fp4_down_kernel     one wave = R rows of W2 for all k experts; lane l owns
//                       words l + 64 i of the row (8 codes each); the fp32 hidden
//                       vector stays fp32 (converter to f32 pairs, fp32 FMA).
#include "decode_common.h"

namespace cachalot {
namespace {

using namespace decode;
constexpr int R_GU = 4;
constexpr int MAXC = 2;   // 64-code chunks per lane, gate/up (D <= 8192)
constexpr int MAXW = 6;   // 8-code words per lane, down (F <= 3072)

__device__ __forceinline__ float fp4_word_dot_bf16(uint32_t w, float scale, const uint32_t* xp, float acc) {
  acc = dot2_bf16(fp4x2_to_bf16x2<0>(w, scale), xp[0], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<1>(w, scale), xp[1], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<2>(w, scale), xp[2], acc);
  acc = dot2_bf16(fp4x2_to_bf16x2<3>(w, scale), xp[3], acc);
  return acc;
}

__global__ void __launch_bounds__(64 * WAVES) fp4_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L,
    const int32_t* __restrict__ slot_table, const int32_t* __restrict__ idx, const float* __restrict__ wts,
    int D, int F, int E, float limit, float* __restrict__ hidden) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const int row0 = (blockIdx.x * WAVES + wave) * R_GU;
  if (row0 >= F) return;
  float* hout = hidden + (size_t)e * F;
  const int slot = expert_slot(slot_table, idx, e, E);
  if (slot < 0) {
    if (lane < R_GU && row0 + lane < F) hout[row0 + lane] = 0.0f;
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const uint4* w1 = reinterpret_cast<const uint4*>(base + L.off[0]);
  const uint8_t* s1 = base + L.off[1];
  const uint4* w3 = reinterpret_cast<const uint4*>(base + L.off[6]);
  const uint8_t* s3 = base + L.off[7];
  const int NC = D / 64;        // 64-code chunks per row (two uint4 each)
  const int SB = D / 32;        // scale blocks per row

  uint32_t xw[MAXC][32];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    const uint4* xp = reinterpret_cast<const uint4*>(x + (size_t)min(c, NC - 1) * 64);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 v = c < NC ? xp[q] : make_uint4(0, 0, 0, 0);
      xw[i][4 * q] = v.x; xw[i][4 * q + 1] = v.y; xw[i][4 * q + 2] = v.z; xw[i][4 * q + 3] = v.w;
    }
  }

  float part[2 * R_GU];
#pragma unroll
  for (int r = 0; r < R_GU; ++r) {
    const int n = min(row0 + r, F - 1);
    float pg = 0.0f, pu = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = lane + 64 * i;
      if (c < NC) {
        const uint4 g0 = w1[((size_t)n * NC + c) * 2];
        const uint4 g1 = w1[((size_t)n * NC + c) * 2 + 1];
        const uint4 u0 = w3[((size_t)n * NC + c) * 2];
        const uint4 u1 = w3[((size_t)n * NC + c) * 2 + 1];
        const float sg0 = e8m0_to_f32(s1[(size_t)n * SB + 2 * c]);
        const float sg1 = e8m0_to_f32(s1[(size_t)n * SB + 2 * c + 1]);
        const float su0 = e8m0_to_f32(s3[(size_t)n * SB + 2 * c]);
        const float su1 = e8m0_to_f32(s3[(size_t)n * SB + 2 * c + 1]);
        pg = fp4_word_dot_bf16(g0.x, sg0, &xw[i][0], pg);
        pu = fp4_word_dot_bf16(u0.x, su0, &xw[i][0], pu);
        pg = fp4_word_dot_bf16(g0.y, sg0, &xw[i][4], pg);
        pu = fp4_word_dot_bf16(u0.y, su0, &xw[i][4], pu);
        pg = fp4_word_dot_bf16(g0.z, sg0, &xw[i][8], pg);
        pu = fp4_word_dot_bf16(u0.z, su0, &xw[i][8], pu);
        pg = fp4_word_dot_bf16(g0.w, sg0, &xw[i][12], pg);
        pu = fp4_word_dot_bf16(u0.w, su0, &xw[i][12], pu);
        pg = fp4_word_dot_bf16(g1.x, sg1, &xw[i][16], pg);
        pu = fp4_word_dot_bf16(u1.x, su1, &xw[i][16], pu);
        pg = fp4_word_dot_bf16(g1.y, sg1, &xw[i][20], pg);
        pu = fp4_word_dot_bf16(u1.y, su1, &xw[i][20], pu);
        pg = fp4_word_dot_bf16(g1.z, sg1, &xw[i][24], pg);
        pu = fp4_word_dot_bf16(u1.z, su1, &xw[i][24], pu);
        pg = fp4_word_dot_bf16(g1.w, sg1, &xw[i][28], pg);
        pu = fp4_word_dot_bf16(u1.w, su1, &xw[i][28], pu);
      }
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
      hout[n] = (silu_f32(g) * u) * wts[e];
    }
  }
}

__global__ void __launch_bounds__(64 * WAVES) fp4_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, const int32_t* __restrict__ slot_table,
    const int32_t* __restrict__ idx, int D, int F, int E, int k, const float* __restrict__ hidden,
    const uint16_t* __restrict__ addend, float* __restrict__ routed, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * WAVES + wave) * R_DN;
  if (row0 >= D) return;
  const int Kw = F / 8;     // 32-bit words per row
  const int SB = F / 32;    // scale blocks per row
  float part[R_DN * KMAX];
#pragma unroll
  for (int i = 0; i < R_DN * KMAX; ++i) part[i] = 0.0f;

#pragma unroll 1
  for (int e = 0; e < k; ++e) {
    const int slot = expert_slot(slot_table, idx, e, E);
    if (slot < 0) continue;
    const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(base + L.off[3]);
    const uint8_t* s2 = base + L.off[4];
    const float4* he = reinterpret_cast<const float4*>(hidden + (size_t)e * F);
    float h[MAXW][8];
#pragma unroll
    for (int i = 0; i < MAXW; ++i) {
      const int j = lane + 64 * i;
      const float4 a = j < Kw ? he[2 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 b = j < Kw ? he[2 * j + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
      h[i][0] = a.x; h[i][1] = a.y; h[i][2] = a.z; h[i][3] = a.w;
      h[i][4] = b.x; h[i][5] = b.y; h[i][6] = b.z; h[i][7] = b.w;
    }
#pragma unroll
    for (int r = 0; r < R_DN; ++r) {
      const int n = min(row0 + r, D - 1);
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < MAXW; ++i) {
        const int j = lane + 64 * i;
        if (j < Kw) {
          const uint32_t wv = w2[(size_t)n * Kw + j];
          const float sc = e8m0_to_f32(s2[(size_t)n * SB + (j >> 2)]);
          const float2_t p0 = fp4x2_to_f32x2<0>(wv, sc);
          const float2_t p1 = fp4x2_to_f32x2<1>(wv, sc);
          const float2_t p2 = fp4x2_to_f32x2<2>(wv, sc);
          const float2_t p3 = fp4x2_to_f32x2<3>(wv, sc);
          acc = __builtin_fmaf(p0[0], h[i][0], acc);
          acc = __builtin_fmaf(p0[1], h[i][1], acc);
          acc = __builtin_fmaf(p1[0], h[i][2], acc);
          acc = __builtin_fmaf(p1[1], h[i][3], acc);
          acc = __builtin_fmaf(p2[0], h[i][4], acc);
          acc = __builtin_fmaf(p2[1], h[i][5], acc);
          acc = __builtin_fmaf(p3[0], h[i][6], acc);
          acc = __builtin_fmaf(p3[1], h[i][7], acc);
        }
      }
#pragma unroll
      for (int ee = 0; ee < KMAX; ++ee)
        if (ee == e) part[r * KMAX + ee] = acc;
    }
  }
  const float red = wave_transpose_sum<R_DN * KMAX>(part, lane);
  finish_rows<false>(red, lane, row0, D, k, addend, routed, out);
}

}  // namespace
}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_fp4_workspace_bytes(int D, int F, int k) {
  (void)D;
  if (F <= 0 || k <= 0) return 0;
  return (size_t)k * (size_t)F * sizeof(float);
}

extern "C" int cachalot_moe_decode_fp4(const uint16_t* x, const uint8_t* pool,
                                       const cachalot_expert_layout* layout, const int32_t* slot_table,
                                       const int32_t* idx, const float* w, int D, int F, int E, int k,
                                       float swiglu_limit, const uint16_t* addend, float* routed, uint16_t* out,
                                       void* workspace, size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  using namespace cachalot::decode;
  CACHALOT_REQUIRE(x && pool && layout && slot_table && idx && w, "moe_decode_fp4: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_fp4: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_fp4: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(E >= 1, "moe_decode_fp4: E=%d", E);
  CACHALOT_REQUIRE(D % 64 == 0 && D >= 64 && D <= 64 * 64 * MAXC,
                   "moe_decode_fp4: D=%d must be a multiple of 64 and <= %d", D, 64 * 64 * MAXC);
  CACHALOT_REQUIRE(F % 32 == 0 && F >= 32 && F <= 8 * 64 * MAXW,
                   "moe_decode_fp4: F=%d must be a multiple of 32 and <= %d", F, 8 * 64 * MAXW);
  const size_t need = cachalot_moe_decode_fp4_workspace_bytes(D, F, k);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(CACHALOT_ESPACE, "moe_decode_fp4: workspace %zu < %zu bytes", workspace_bytes, need);
  Layout L;
  static const int used[6] = {0, 1, 3, 4, 6, 7};
  int rc = make_layout(layout, 6, used, L, "moe_decode_fp4");
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  float* hidden = static_cast<float*>(workspace);
  dim3 g1((F + R_GU * WAVES - 1) / (R_GU * WAVES), k);
  hipLaunchKernelGGL(fp4_gate_up_kernel, g1, dim3(64 * WAVES), 0, s, x, pool, L, slot_table, idx, w, D, F, E,
                     swiglu_limit, hidden);
  rc = check_launch("fp4_gate_up_kernel");
  if (rc) return rc;
  dim3 g2((D + R_DN * WAVES - 1) / (R_DN * WAVES));
  hipLaunchKernelGGL(fp4_down_kernel, g2, dim3(64 * WAVES), 0, s, pool, L, slot_table, idx, D, F, E, k, hidden,
                     addend, routed, out);
  return check_launch("fp4_down_kernel");
}
