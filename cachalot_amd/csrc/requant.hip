// FP4 (E2M1 + E8M0 block-32) weights -> 2-bit affine g128 (MLX layout), the
// searched fit of benchmarks/quant_affine.py (_quantize :130-133, _error
// :136-140, fit_minmax :157-167, SHRINKS :174, fit_search :177-205,
// quantize_affine :330-359), on the GPU.
//
// One thread per 128-element group of a weight row: the group's FP4 values are
// decoded exactly to fp32 by the hardware converter, then
//   lo, hi, mid = (lo + hi) / 2; the min/max fit scale = max((hi - lo) / 3, 1e-8),
//   bias = lo; each of the 24 shrunk ranges (s_lo, s_hi in SHRINKS, (1, 1)
//   skipped, in order) replaces the best when its error is strictly smaller;
//   error = sum over the group in index order of (scale q + bias - w)^2 with
//   q = clip(rint((w - bias) / scale), 0, 3);
// then scale and bias are rounded (RNE) to the bank's storage type, bf16 or
// fp16, the codes recomputed against them (an fp16 scale that rounds to zero,
// a constant group, gives code 0)
// and packed 16 per word, low field first.  Every operation is a single fp32
// operation in the written order (the library is built without contraction),
// so the result equals a float32 evaluation in the same order bit for bit.
// K not a multiple of 128 (w2 at d_ff = 2880): the last group fits its real
// elements only and its padding codes are 0.
#include "common.h"

namespace cachalot {
namespace requant {

constexpr int GROUP = 128;
constexpr int NSHRINK = 5;
__constant__ float kShrinks[NSHRINK] = {1.0f, 0.925f, 0.85f, 0.775f, 0.7f};

struct Args {
  const uint8_t* w;      // [N, K/2] packed E2M1, low nibble first
  const uint8_t* s;      // [N, K/32] E8M0
  int N, K;
  uint32_t* q;           // [N, G * 8] 2-bit codes
  uint16_t* scales;      // [N, G] bf16 or fp16 (f16)
  uint16_t* biases;      // [N, G] bf16 or fp16
  bool f16;
};

__device__ __forceinline__ float level(float w, float scale, float bias) {
  return fminf(fmaxf(rintf((w - bias) / scale), 0.0f), 3.0f);
}

__device__ __forceinline__ float group_error(const float (&w)[GROUP], int nvalid, float scale, float bias) {
  float err = 0.0f;
#pragma unroll
  for (int i = 0; i < GROUP; ++i) {
    const float d = scale * level(w[i], scale, bias) + bias - w[i];
    if (i < nvalid) err = err + d * d;
  }
  return err;
}

__global__ __launch_bounds__(256) void requant_fp4_q2_kernel(Args p) {
  const int G = (p.K + GROUP - 1) / GROUP;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)p.N * G) return;
  const int n = (int)(gid / G), g = (int)(gid % G);
  const int nvalid = min(GROUP, p.K - g * GROUP);
  const uint8_t* wrow = p.w + (size_t)n * (p.K / 2) + g * (GROUP / 2);
  const uint8_t* srow = p.s + (size_t)n * (p.K / 32) + g * (GROUP / 32);

  float w[GROUP];
#pragma unroll
  for (int b = 0; b < GROUP / 32; ++b) {           // 32-element blocks: 16 code bytes + one scale
    uint4 c = make_uint4(0, 0, 0, 0);
    float sc = 1.0f;
    if (b * 32 < nvalid) {
      c = *reinterpret_cast<const uint4*>(wrow + b * 16);
      sc = e8m0_to_f32(srow[b]);
    }
    const uint32_t words[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2_t v0 = fp4x2_to_f32x2<0>(words[j], sc);
      const float2_t v1 = fp4x2_to_f32x2<1>(words[j], sc);
      const float2_t v2 = fp4x2_to_f32x2<2>(words[j], sc);
      const float2_t v3 = fp4x2_to_f32x2<3>(words[j], sc);
      float* o = w + b * 32 + j * 8;
      o[0] = v0[0]; o[1] = v0[1]; o[2] = v1[0]; o[3] = v1[1];
      o[4] = v2[0]; o[5] = v2[1]; o[6] = v3[0]; o[7] = v3[1];
    }
  }

  float lo = INFINITY, hi = -INFINITY;
#pragma unroll
  for (int i = 0; i < GROUP; ++i)
    if (i < nvalid) {
      lo = fminf(lo, w[i]);
      hi = fmaxf(hi, w[i]);
    }
  const float mid = (lo + hi) / 2.0f;
  float best_s = fmaxf((hi - lo) / 3.0f, 1e-8f), best_b = lo;
  float best = group_error(w, nvalid, best_s, best_b);
  for (int a = 0; a < NSHRINK; ++a) {
    for (int c = 0; c < NSHRINK; ++c) {
      if (a == 0 && c == 0) continue;
      const float new_lo = mid + (lo - mid) * kShrinks[a];
      const float new_hi = mid + (hi - mid) * kShrinks[c];
      const float s = fmaxf((new_hi - new_lo) / 3.0f, 1e-8f);
      const float err = group_error(w, nvalid, s, new_lo);
      if (err < best) {
        best_s = s;
        best_b = new_lo;
      }
      best = fminf(err, best);
    }
  }

  const uint16_t sb = p.f16 ? f32_to_f16(best_s) : f32_to_bf16(best_s);
  const uint16_t bb = p.f16 ? f32_to_f16(best_b) : f32_to_bf16(best_b);
  const float s16 = scale_bits_to_f32(sb, p.f16), b16 = scale_bits_to_f32(bb, p.f16);
  uint32_t words[GROUP / 16];
#pragma unroll
  for (int j = 0; j < GROUP / 16; ++j) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int k = 16 * j + i;
      const uint32_t q = k < nvalid && s16 != 0.0f ? (uint32_t)level(w[k], s16, b16) : 0u;
      v |= q << (2 * i);
    }
    words[j] = v;
  }
  uint4* qdst = reinterpret_cast<uint4*>(p.q + (size_t)n * G * 8 + g * 8);
  qdst[0] = make_uint4(words[0], words[1], words[2], words[3]);
  qdst[1] = make_uint4(words[4], words[5], words[6], words[7]);
  p.scales[(size_t)n * G + g] = sb;
  p.biases[(size_t)n * G + g] = bb;
}

}  // namespace requant
}  // namespace cachalot

using namespace cachalot;

extern "C" int cachalot_requant_fp4_to_q2(const uint8_t* w_fp4, const uint8_t* s_fp4, int N, int K, uint32_t* q,
                                          uint16_t* scales, uint16_t* biases, int scale_dtype,
                                          cachalot_stream_t stream) {
  CACHALOT_REQUIRE(w_fp4 && s_fp4 && q && scales && biases, "requant_fp4_to_q2: null pointer");
  CACHALOT_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "requant_fp4_to_q2: N=%d, K=%d (K a positive multiple of 32)", N, K);
  CACHALOT_REQUIRE(((uintptr_t)w_fp4 & 15u) == 0 && ((uintptr_t)q & 15u) == 0,
                   "requant_fp4_to_q2: w_fp4 and q must be 16-byte aligned");
  const long groups = (long)N * ((K + requant::GROUP - 1) / requant::GROUP);
  CACHALOT_REQUIRE(scale_dtype == CACHALOT_SCALE_BF16 || scale_dtype == CACHALOT_SCALE_F16,
                   "requant_fp4_to_q2: scale_dtype %d (0 = bf16, 1 = fp16)", scale_dtype);
  requant::Args a{w_fp4, s_fp4, N, K, q, scales, biases, scale_dtype == CACHALOT_SCALE_F16};
  hipLaunchKernelGGL(requant::requant_fp4_q2_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("requant_fp4_to_q2");
}
