// Dense dequantisation kernels: the GPU side of the bit-exact weight checks.
//
// FP4: value = E2M1(nibble) * 2^(e - 127) (src/cachalot/model/fp4.py:67-109,
// fp4_dequant_metal.py:10-40), low nibble first.  Produced by the same gfx950
// converters the decode / prefill kernels use (f32 or, with as_bf16, the bf16
// form), so a bit-exact match here pins the conversion those kernels rely on.
// 2-bit affine: value = fl(fl(s * q) + b) with q extracted exactly as the
// decode kernels do (spread into FP4 nibbles, converted to bf16).
#include "common.h"

namespace cachalot {
namespace {

// one thread per 32-bit word of packed codes (8 values)
__global__ void dequant_fp4_kernel(const uint32_t* __restrict__ packed, const uint8_t* __restrict__ scales, int N,
                                   int K, int as_bf16, float* __restrict__ out) {
  const int64_t words = (int64_t)N * (K / 8);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t n = i / (K / 8);
  const int64_t j = i % (K / 8);
  const float sc = e8m0_to_f32(scales[n * (K / 32) + j / 4]);
  const uint32_t w = packed[i];
  float v[8];
  if (as_bf16) {
    const uint32_t p[4] = {fp4x2_to_bf16x2<0>(w, sc), fp4x2_to_bf16x2<1>(w, sc), fp4x2_to_bf16x2<2>(w, sc),
                           fp4x2_to_bf16x2<3>(w, sc)};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      v[2 * b] = __uint_as_float(p[b] << 16);
      v[2 * b + 1] = __uint_as_float(p[b] & 0xffff0000u);
    }
  } else {
    const float2_t p[4] = {fp4x2_to_f32x2<0>(w, sc), fp4x2_to_f32x2<1>(w, sc), fp4x2_to_f32x2<2>(w, sc),
                           fp4x2_to_f32x2<3>(w, sc)};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      v[2 * b] = p[b][0];
      v[2 * b + 1] = p[b][1];
    }
  }
  float4* o = reinterpret_cast<float4*>(out + n * K + j * 8);
  o[0] = make_float4(v[0], v[1], v[2], v[3]);
  o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// one thread per 32-bit word of codes (16 values)
__global__ void dequant_q2_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
                                  const uint16_t* __restrict__ biases, int N, int K, int row_words, int groups,
                                  int group, bool f16, float* __restrict__ out) {
  const int kw = (K + 15) / 16;
  const int64_t total = (int64_t)N * kw;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t n = i / kw;
  const int j = (int)(i % kw);
  const uint32_t word = w[n * row_words + j];
  const uint32_t ev = word & 0x33333333u;
  const uint32_t od = (word >> 2) & 0x33333333u;
  const uint32_t pe[4] = {fp4x2_to_bf16x2<0>(ev, 2.0f), fp4x2_to_bf16x2<1>(ev, 2.0f), fp4x2_to_bf16x2<2>(ev, 2.0f),
                          fp4x2_to_bf16x2<3>(ev, 2.0f)};
  const uint32_t po[4] = {fp4x2_to_bf16x2<0>(od, 2.0f), fp4x2_to_bf16x2<1>(od, 2.0f), fp4x2_to_bf16x2<2>(od, 2.0f),
                          fp4x2_to_bf16x2<3>(od, 2.0f)};
  float q[16];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    q[4 * b] = __uint_as_float(pe[b] << 16);
    q[4 * b + 2] = __uint_as_float(pe[b] & 0xffff0000u);
    q[4 * b + 1] = __uint_as_float(po[b] << 16);
    q[4 * b + 3] = __uint_as_float(po[b] & 0xffff0000u);
  }
  const int g = (j * 16) / group;
  const float s = scale_bits_to_f32(scales[n * groups + g], f16);
  const float b = scale_bits_to_f32(biases[n * groups + g], f16);
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int k = j * 16 + t;
    if (k < K) out[n * K + k] = s * q[t] + b;
  }
}

}  // namespace
}  // namespace cachalot

extern "C" int cachalot_dequant_fp4(const uint8_t* packed, const uint8_t* scales, int N, int K, int as_bf16,
                                    float* out, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(packed && scales && out, "dequant_fp4: null pointer");
  CACHALOT_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "dequant_fp4: K=%d must be divisible by block_size=32", K);
  const int64_t words = (int64_t)N * (K / 8);
  const int threads = 256;
  hipLaunchKernelGGL(dequant_fp4_kernel, dim3((unsigned)((words + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(packed), scales, N, K, as_bf16, out);
  return check_launch("dequant_fp4_kernel");
}

extern "C" int cachalot_dequant_q2(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                                   int row_words, int groups, int group, int scale_dtype, float* out,
                                   cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(w && scales && biases && out, "dequant_q2: null pointer");
  CACHALOT_REQUIRE(N >= 1 && K >= 1 && group >= 16 && group % 16 == 0, "dequant_q2: bad shape N=%d K=%d group=%d",
                   N, K, group);
  CACHALOT_REQUIRE(row_words * 16 >= K && groups * group >= K, "dequant_q2: row_words %d / groups %d too small",
                   row_words, groups);
  CACHALOT_REQUIRE(scale_dtype == CACHALOT_SCALE_BF16 || scale_dtype == CACHALOT_SCALE_F16,
                   "dequant_q2: scale_dtype %d (0 = bf16, 1 = fp16)", scale_dtype);
  const int64_t total = (int64_t)N * ((K + 15) / 16);
  const int threads = 256;
  hipLaunchKernelGGL(dequant_q2_kernel, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, w, scales, biases, N, K, row_words, groups, group,
                     scale_dtype == CACHALOT_SCALE_F16, out);
  return check_launch("dequant_q2_kernel");
}
