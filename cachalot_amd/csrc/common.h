// Shared device helpers and C-ABI error plumbing for libcachalot_amd.
//
// Every translation unit is compiled for gfx950 only, with
// -ffp-contract=off (so the order and rounding of float operations is the
// one written, which the router's bit-exact contract relies on) and with
// packed-FP32 code generation disabled.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/cachalot_amd.h"

namespace cachalot {

// ---------------------------------------------------------------- errors ---
// Thread-local last error message, returned by cachalot_last_error().
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

#define CACHALOT_REQUIRE(cond, ...)                                          \
  do {                                                                      \
    if (!(cond)) return ::cachalot::fail(CACHALOT_EINVAL, __VA_ARGS__);     \
  } while (0)

// ------------------------------------------------------------------ bf16 ---
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float float2_t;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (quiet NaN preserved).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t u) {
  return __builtin_bit_cast(bf16x2_t, u);
}

// fp32 dot of two bf16 pairs accumulated into c (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a), as_bf16x2(b), c, false);
}

// Two FP4 E2M1 nibbles of byte `sel` of `w` -> two bf16 (low nibble first),
// multiplied by `scale` (a power of two).  Hardware converter of gfx950.
template <int sel>
__device__ __forceinline__ uint32_t fp4x2_to_bf16x2(uint32_t w, float scale) {
  auto r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, sel);
  return __builtin_bit_cast(uint32_t, r);
}

template <int sel>
__device__ __forceinline__ float2_t fp4x2_to_f32x2(uint32_t w, float scale) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, sel);
}

// E8M0 exponent byte -> fp32 2^(raw-127) (raw 0 gives 2^-127, a subnormal).
__device__ __forceinline__ float e8m0_to_f32(uint32_t raw) {
  return raw == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(raw << 23);
}

// ------------------------------------------------------- wave reductions ---
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Full wave64 sum (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}

// Transposed reduction of N (power of two, <= 64) per-lane values:
// afterwards lane L holds, in v[0], the wave-wide sum of value index
// (L >> (6 - log2 N)) -- i.e. value i ends in lanes [i*64/N, (i+1)*64/N).
template <int N>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[N], int lane) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
  int n = N;
  int bit = 32;
#pragma unroll
  for (int step = 0; (1 << step) < N; ++step) {
    const int half = n >> 1;
    const bool hi = (lane & bit) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      if (i < half) {
        float keep = hi ? v[i + half] : v[i];
        float send = hi ? v[i] : v[i + half];
        v[i] = keep + shfl_xor_f(send, bit);
      }
    }
    n = half;
    bit >>= 1;
  }
  float r = v[0];
  for (; bit >= 1; bit >>= 1) r += shfl_xor_f(r, bit);
  return r;
}

}  // namespace cachalot
