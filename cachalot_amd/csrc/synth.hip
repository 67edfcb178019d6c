// Seeded synthetic fill (test and benchmark data, written straight into HBM).
//
// rand(key, i) = fmix64(key + (i + 1) * GAMMA), SplitMix64's finaliser
// (Steele, Lea & Flood, OOPSLA 2014).  Kinds and their exact arithmetic are
// fixed so that a host re-implementation can regenerate any element bit for
// bit: every float step is one IEEE operation in double, then one rounding
// to fp32 (and RNE to bf16 or fp16).
#include "common.h"

namespace cachalot {
namespace {

constexpr uint64_t GAMMA = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t fmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ double irwin_hall(uint64_t r, double c) {
  double s = (double)(r & 0xFFFF) + (double)((r >> 16) & 0xFFFF);
  s = s + (double)((r >> 32) & 0xFFFF);
  s = s + (double)((r >> 48) & 0xFFFF);
  return (s - 131070.0) * c;
}

__global__ void fill_kernel(void* dst, int64_t n, int64_t start, uint64_t key, int kind, double p0,
                            double p1, int64_t row_total, int64_t row_valid) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t ctr = (uint64_t)(start + i);
    const uint64_t r = fmix64(key + (ctr + 1) * GAMMA);
    switch (kind) {
      case 0: {
        uint32_t v = (uint32_t)r;
        if (row_total > 0 && (int64_t)(ctr % (uint64_t)row_total) >= row_valid) v = 0;
        ((uint32_t*)dst)[i] = v;
        break;
      }
      case 1: {
        const uint64_t span = (uint64_t)(p1 - p0) + 1;
        ((uint8_t*)dst)[i] = (uint8_t)((uint64_t)p0 + (r >> 32) % span);
        break;
      }
      case 2: {
        const double t = (double)(r >> 40) * 0x1p-24;
        const double v = p0 + p1 * t;
        ((uint16_t*)dst)[i] = f32_to_bf16((float)v);
        break;
      }
      case 3:
        ((uint16_t*)dst)[i] = f32_to_bf16((float)irwin_hall(r, p1));
        break;
      case 5: {
        const double t = (double)(r >> 40) * 0x1p-24;
        ((uint16_t*)dst)[i] = f32_to_f16((float)(p0 + p1 * t));
        break;
      }
      case 6:
        ((uint16_t*)dst)[i] = f32_to_f16((float)irwin_hall(r, p1));
        break;
      default:
        ((float*)dst)[i] = (float)irwin_hall(r, p1);
        break;
    }
  }
}

}  // namespace
}  // namespace cachalot

extern "C" int cachalot_fill_synthetic(void* dst, int64_t n, int64_t start, uint64_t key, int kind,
                                       double p0, double p1, int64_t row_total, int64_t row_valid,
                                       cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(dst != nullptr || n == 0, "fill: null destination");
  CACHALOT_REQUIRE(n >= 0 && start >= 0, "fill: negative size");
  CACHALOT_REQUIRE(kind >= 0 && kind <= 6, "fill: unknown kind %d", kind);
  CACHALOT_REQUIRE(kind != 1 || (p0 >= 0 && p1 <= 255 && p0 <= p1), "fill: E8M0 range [%g, %g]", p0, p1);
  if (n == 0) return CACHALOT_OK;
  // kinds 3/4/6 take the Irwin-Hall scale c = sigma / std in p1 (the host computes it)
  const int threads = 256;
  int64_t blocks = (n + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream, dst, n,
                     start, key, kind, p0, p1, row_total, row_valid);
  return check_launch("cachalot_fill_synthetic");
}
