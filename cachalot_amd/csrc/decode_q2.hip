// Decode (one token) over a 2-bit affine g128 expert bank.
//
// Reference: src/cachalot/model/expert_affine.py:65-81 (rounding points),
// :117-152 (topk_core: experts summed in route order), moe_layer_metal.py:
// 93-130 (the traced block), mx.quantized_matmul's group formula
// s * sum(x q) + b * sum(x) (MLX qdot, as copied at minimax/codes_qmv.py:86-100).
//
// Two launches per token-layer:
//   q2_gate_up_kernel  one wave = R rows of one expert; each lane owns one
//                      64-code uint4 chunk of the row (K = 4096 -> the whole row
//                      in one coalesced 1 KiB wave load per matrix).  Codes are
//                      spread into FP4 nibbles (q in 0..3 is the E2M1 code of
//                      q/2) and turned into bf16 pairs by the gfx950 converter,
//                      then dotted with pre-paired bf16 activations
//                      (v_dot2c_f32_bf16, exact products, fp32 accumulation).
//                      Epilogue: bf16(g), bf16(u), clamp, bf16(silu(g)*u*w_e),
//                      written into the workspace in the pair order the down
//                      kernel consumes.
//   q2_down_kernel     one wave = R rows of W2 for all k experts; lane l owns
//                      words l, l+64, l+128 of the row (K = 2880 -> 180 words);
//                      per (row, expert) partials are reduced with one
//                      transposed wave reduction, rounded to bf16 per expert
//                      and summed in route order, + addend, -> fp32 / bf16.
#include "decode_common.h"

namespace cachalot {
namespace {

using namespace decode;
constexpr int R_GU = 4;     // rows per wave, gate/up
constexpr int MAXC = 2;     // max 64-code chunks per lane in gate/up (D <= 8192)
constexpr int MAXW = 3;     // max words per lane in down (F <= 3072)

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

// Build E/O pairs from 4 natural-order words holding (v0,v1),(v2,v3),(v4,v5),(v6,v7)
// -> E = (v0,v2),(v4,v6); O = (v1,v3),(v5,v7).
__device__ __forceinline__ void make_pairs(uint32_t a, uint32_t b, uint32_t& e, uint32_t& o) {
  e = (a & 0xffffu) | (b << 16);
  o = (a >> 16) | (b & 0xffff0000u);
}

constexpr uint32_t BF16_ONES = 0x3f803f80u;


__global__ void __launch_bounds__(64 * WAVES) q2_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L,
    const int32_t* __restrict__ slot_table, const int32_t* __restrict__ idx, const float* __restrict__ wts,
    int D, int F, int E, int group, float limit, uint16_t* __restrict__ hp) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const int row0 = (blockIdx.x * WAVES + wave) * R_GU;
  const int Fw = F / 16;
  uint16_t* hout = hp + (size_t)e * Fw * 16;
  if (row0 >= F) return;
  const int slot = expert_slot(slot_table, idx, e, E);
  if (slot < 0) {
    if (lane < R_GU && row0 + lane < F) {
      const int n = row0 + lane;
      hout[(n >> 4) * 16 + pair_pos(n & 15)] = 0;
    }
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const int words = D / 16;   // row stride (D is a whole number of groups)
  const int G = D / group;
  const uint4* w1 = reinterpret_cast<const uint4*>(base + L.off[0]);
  const uint16_t* s1 = reinterpret_cast<const uint16_t*>(base + L.off[1]);
  const uint16_t* b1 = reinterpret_cast<const uint16_t*>(base + L.off[2]);
  const uint4* w3 = reinterpret_cast<const uint4*>(base + L.off[6]);
  const uint16_t* s3 = reinterpret_cast<const uint16_t*>(base + L.off[7]);
  const uint16_t* b3 = reinterpret_cast<const uint16_t*>(base + L.off[8]);
  const int NC = D / 64;

  // activation pairs and sums for this lane's chunks
  uint32_t xe[MAXC][4][4], xo[MAXC][4][4];
  float xs[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    xs[i] = 0.0f;
    if (c < NC) {
      const uint4* xp = reinterpret_cast<const uint4*>(x + (size_t)c * 64);
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // word j covers x[16j .. 16j+16)
        const uint4 a = xp[2 * j];
        const uint4 b = xp[2 * j + 1];
        make_pairs(a.x, a.y, xe[i][j][0], xo[i][j][0]);
        make_pairs(a.z, a.w, xe[i][j][1], xo[i][j][1]);
        make_pairs(b.x, b.y, xe[i][j][2], xo[i][j][2]);
        make_pairs(b.z, b.w, xe[i][j][3], xo[i][j][3]);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = dot2_bf16(xe[i][j][q], BF16_ONES, s);
          s = dot2_bf16(xo[i][j][q], BF16_ONES, s);
        }
        xs[i] = xs[i] + s;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) xe[i][j][q] = xo[i][j][q] = 0u;
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
        const uint4 vg = w1[(size_t)n * (words / 4) + c];
        const uint4 vu = w3[(size_t)n * (words / 4) + c];
        const int g = (c * 64) / group;
        const float sg = bf16_to_f32(s1[(size_t)n * G + g]);
        const float bg = bf16_to_f32(b1[(size_t)n * G + g]);
        const float su = bf16_to_f32(s3[(size_t)n * G + g]);
        const float bu = bf16_to_f32(b3[(size_t)n * G + g]);
        float dg = 0.0f, du = 0.0f;
        dg = q2_word_dot(vg.x, xe[i][0], xo[i][0], dg);
        du = q2_word_dot(vu.x, xe[i][0], xo[i][0], du);
        dg = q2_word_dot(vg.y, xe[i][1], xo[i][1], dg);
        du = q2_word_dot(vu.y, xe[i][1], xo[i][1], du);
        dg = q2_word_dot(vg.z, xe[i][2], xo[i][2], dg);
        du = q2_word_dot(vu.z, xe[i][2], xo[i][2], du);
        dg = q2_word_dot(vg.w, xe[i][3], xo[i][3], dg);
        du = q2_word_dot(vu.w, xe[i][3], xo[i][3], du);
        pg = pg + (sg * dg + bg * xs[i]);
        pu = pu + (su * du + bu * xs[i]);
      }
    }
    part[2 * r] = pg;
    part[2 * r + 1] = pu;
  }
  // value 2r+v ends in lanes [8(2r+v), 8(2r+v)+8)
  const float red = wave_transpose_sum<2 * R_GU>(part, lane);
  const float up = __shfl(red, lane + 8, 64);
  if ((lane & 15) == 0) {
    const int r = lane >> 4;
    const int n = row0 + r;
    if (n < F) {
      float g = round_bf16(red);
      float u = round_bf16(up);
      if (limit > 0.0f) {
        u = fminf(fmaxf(u, -limit), limit);
        g = fminf(g, limit);
      }
      const float h = (silu_f32(g) * u) * wts[e];
      hout[(n >> 4) * 16 + pair_pos(n & 15)] = f32_to_bf16(h);
    }
  }
}

__global__ void __launch_bounds__(64 * WAVES) q2_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, const int32_t* __restrict__ slot_table,
    const int32_t* __restrict__ idx, int D, int F, int E, int k, int group, const uint16_t* __restrict__ hp,
    const uint16_t* __restrict__ addend, float* __restrict__ routed, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * WAVES + wave) * R_DN;
  if (row0 >= D) return;
  const int Kw = F / 16;                   // valid words per row
  const int G = (F + group - 1) / group;   // groups per row (last may be partial)
  const int stride = G * group / 16;       // stored words per row
  float part[R_DN * KMAX];
#pragma unroll
  for (int i = 0; i < R_DN * KMAX; ++i) part[i] = 0.0f;

#pragma unroll 1
  for (int e = 0; e < k; ++e) {
    const int slot = expert_slot(slot_table, idx, e, E);
    if (slot < 0) continue;
    const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(base + L.off[3]);
    const uint16_t* s2 = reinterpret_cast<const uint16_t*>(base + L.off[4]);
    const uint16_t* b2 = reinterpret_cast<const uint16_t*>(base + L.off[5]);
    const uint4* hpe = reinterpret_cast<const uint4*>(hp + (size_t)e * Kw * 16);
    uint32_t he[MAXW][4], ho[MAXW][4];
    float hs[MAXW];
#pragma unroll
    for (int i = 0; i < MAXW; ++i) {
      const int j = lane + 64 * i;
      hs[i] = 0.0f;
      if (j < Kw) {
        const uint4 a = hpe[2 * j];
        const uint4 b = hpe[2 * j + 1];
        he[i][0] = a.x; he[i][1] = a.y; he[i][2] = a.z; he[i][3] = a.w;
        ho[i][0] = b.x; ho[i][1] = b.y; ho[i][2] = b.z; ho[i][3] = b.w;
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = dot2_bf16(he[i][q], BF16_ONES, s);
          s = dot2_bf16(ho[i][q], BF16_ONES, s);
        }
        hs[i] = s;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) he[i][q] = ho[i][q] = 0u;
      }
    }
#pragma unroll
    for (int r = 0; r < R_DN; ++r) {
      const int n = min(row0 + r, D - 1);
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < MAXW; ++i) {
        const int j = lane + 64 * i;
        if (j < Kw) {
          const uint32_t wv = w2[(size_t)n * stride + j];
          const int g = (j * 16) / group;
          const float s = bf16_to_f32(s2[(size_t)n * G + g]);
          const float b = bf16_to_f32(b2[(size_t)n * G + g]);
          const float d = q2_word_dot(wv, he[i], ho[i], 0.0f);
          acc = acc + (s * d + b * hs[i]);
        }
      }
      // e < KMAX is guaranteed by the host
#pragma unroll
      for (int ee = 0; ee < KMAX; ++ee)
        if (ee == e) part[r * KMAX + ee] = acc;
    }
  }
  const float red = wave_transpose_sum<R_DN * KMAX>(part, lane);
  finish_rows<true>(red, lane, row0, D, k, addend, routed, out);
}

}  // namespace
}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_q2_workspace_bytes(int D, int F, int k) {
  (void)D;
  if (F <= 0 || k <= 0) return 0;
  return (size_t)k * (size_t)((F + 15) / 16) * 16 * sizeof(uint16_t);
}

extern "C" int cachalot_moe_decode_q2(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                                      const int32_t* slot_table, const int32_t* idx, const float* w, int D, int F,
                                      int E, int k, int group, float swiglu_limit, const uint16_t* addend,
                                      float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                      cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(x && pool && layout && slot_table && idx && w, "moe_decode_q2: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_q2: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_q2: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(E >= 1, "moe_decode_q2: E=%d", E);
  CACHALOT_REQUIRE(group == 64 || group == 128, "moe_decode_q2: group_size %d (64 or 128)", group);
  CACHALOT_REQUIRE(D % group == 0 && D >= 64 && D <= 64 * 64 * MAXC,
                   "moe_decode_q2: D=%d must be a multiple of group %d and <= %d", D, group, 64 * 64 * MAXC);
  CACHALOT_REQUIRE(F % 16 == 0 && F >= 16 && F <= 16 * 64 * MAXW,
                   "moe_decode_q2: F=%d must be a multiple of 16 and <= %d", F, 16 * 64 * MAXW);
  const size_t need = cachalot_moe_decode_q2_workspace_bytes(D, F, k);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(CACHALOT_ESPACE, "moe_decode_q2: workspace %zu < %zu bytes", workspace_bytes, need);
  Layout L;
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  int rc = make_layout(layout, 9, used, L, "moe_decode_q2");
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  uint16_t* hp = static_cast<uint16_t*>(workspace);
  dim3 g1((F + R_GU * WAVES - 1) / (R_GU * WAVES), k);
  hipLaunchKernelGGL(q2_gate_up_kernel, g1, dim3(64 * WAVES), 0, s, x, pool, L, slot_table, idx, w, D, F, E, group,
                     swiglu_limit, hp);
  rc = check_launch("q2_gate_up_kernel");
  if (rc) return rc;
  dim3 g2((D + R_DN * WAVES - 1) / (R_DN * WAVES));
  hipLaunchKernelGGL(q2_down_kernel, g2, dim3(64 * WAVES), 0, s, pool, L, slot_table, idx, D, F, E, k, group, hp,
                     addend, routed, out);
  return check_launch("q2_down_kernel");
}
