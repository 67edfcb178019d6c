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

// Round-to-nearest-even fp32 -> fp16 bits (the hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// A 2-bit bank's scale or bias as stored: bf16 bits, or fp16 bits when `f16`
// (both convert to fp32 exactly).
__device__ __forceinline__ float scale_bits_to_f32(uint16_t b, bool f16) {
  return f16 ? (float)__builtin_bit_cast(_Float16, b) : bf16_to_f32(b);
}

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

// ------------------------------------------------------------- barriers ---
// Workgroup barrier that orders LDS only.  __syncthreads() is a workgroup
// release/acquire fence on all memory, and since gfx9 counts loads and stores
// in one counter that fence waits for every outstanding global load; kernels
// that keep weight loads in flight across a barrier use this one instead and
// wait for their own global traffic explicitly where another wave consumes it.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ------------------------------------------------------- wave reductions ---
// Lane exchanges without the LDS crossbar: DPP for partners inside a row of 16
// lanes, the gfx950 permlane swaps across rows.  xorN(v) returns the value of
// lane (lane ^ N); mirror8 returns lane (lane ^ 7) within each group of 8.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t xor1_u32(uint32_t v) { return dpp_u32<0xB1>(v); }    // quad_perm [1,0,3,2]
__device__ __forceinline__ uint32_t xor2_u32(uint32_t v) { return dpp_u32<0x4E>(v); }    // quad_perm [2,3,0,1]
__device__ __forceinline__ uint32_t mirror8_u32(uint32_t v) { return dpp_u32<0x141>(v); } // row_half_mirror
__device__ __forceinline__ uint32_t mirror16_u32(uint32_t v) { return dpp_u32<0x140>(v); } // row_mirror
__device__ __forceinline__ uint32_t xor8_u32(uint32_t v) { return dpp_u32<0x128>(v); }   // row_ror:8
__device__ __forceinline__ uint32_t xor4_u32(uint32_t v) { return (uint32_t)__shfl_xor((int)v, 4, 64); }
__device__ __forceinline__ uint32_t xor16_u32(uint32_t v) {
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (__lane_id() & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32_u32(uint32_t v) {
  auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (__lane_id() & 32) ? r[0] : r[1];
}
template <int M>
__device__ __forceinline__ uint32_t xor_u32(uint32_t v) {
  if constexpr (M == 1) return xor1_u32(v);
  else if constexpr (M == 2) return xor2_u32(v);
  else if constexpr (M == 4) return xor4_u32(v);
  else if constexpr (M == 8) return xor8_u32(v);
  else if constexpr (M == 16) return xor16_u32(v);
  else return xor32_u32(v);
}
template <int M>
__device__ __forceinline__ float xor_f(float v) {
  return __uint_as_float(xor_u32<M>(__float_as_uint(v)));
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Full wave64 sum, every lane ends with the same value.  Partners: 1, 2 (exact
// xor), then the mirror of the other half of 8 and of 16 (after the earlier
// steps those lanes hold the same value as the xor-4 / xor-8 partner), then 16
// and 32.  Bit-identical to the xor butterfly 1, 2, 4, 8, 16, 32.
__device__ __forceinline__ float wave_sum(float v) {
  v = v + __uint_as_float(xor1_u32(__float_as_uint(v)));
  v = v + __uint_as_float(xor2_u32(__float_as_uint(v)));
  v = v + __uint_as_float(mirror8_u32(__float_as_uint(v)));
  v = v + __uint_as_float(mirror16_u32(__float_as_uint(v)));
  v = v + xor_f<16>(v);
  v = v + xor_f<32>(v);
  return v;
}

// Sum over the 16 lanes of each row (xor 1, 2, then mirrors), bit-identical to
// the xor butterfly 1, 2, 4, 8.
__device__ __forceinline__ float row16_sum(float v) {
  v = v + __uint_as_float(xor1_u32(__float_as_uint(v)));
  v = v + __uint_as_float(xor2_u32(__float_as_uint(v)));
  v = v + __uint_as_float(mirror8_u32(__float_as_uint(v)));
  v = v + __uint_as_float(mirror16_u32(__float_as_uint(v)));
  return v;
}

// Butterfly 32, 16, 8, 4, 2, 1 as the router contract states it (a + partner).
__device__ __forceinline__ float wave_sum_xor_desc(float v) {
  v = v + xor_f<32>(v);
  v = v + xor_f<16>(v);
  v = v + xor_f<8>(v);
  v = v + xor_f<4>(v);
  v = v + xor_f<2>(v);
  v = v + xor_f<1>(v);
  return v;
}

// Transposed reduction of N (power of two, <= 8) per-lane values: afterwards
// every lane of [i*64/N, (i+1)*64/N) holds the wave-wide sum of value i.
// The transposing steps use exact xor partners 32, 16, 8; the rest is a row sum.
template <int N>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[N], int lane) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8, "N must be 1, 2, 4 or 8");
  if constexpr (N >= 2) {
    const bool hi = (lane & 32) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float keep = hi ? v[i + N / 2] : v[i];
      const float send = hi ? v[i] : v[i + N / 2];
      v[i] = keep + xor_f<32>(send);
    }
  }
  if constexpr (N >= 4) {
    const bool hi = (lane & 16) != 0;
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const float keep = hi ? v[i + N / 4] : v[i];
      const float send = hi ? v[i] : v[i + N / 4];
      v[i] = keep + xor_f<16>(send);
    }
  }
  if constexpr (N >= 8) {
    const bool hi = (lane & 8) != 0;
    const float keep = hi ? v[1] : v[0];
    const float send = hi ? v[0] : v[1];
    v[0] = keep + xor_f<8>(send);
  }
  float r = v[0];
  if constexpr (N == 1) return wave_sum(r);
  if constexpr (N == 2) {  // lanes of a 32-half: sum over bits 4..0
    r = row16_sum(r);
    return r + xor_f<16>(r);
  }
  if constexpr (N == 4) return row16_sum(r);
  // N == 8: sum over bits 2..0 (groups of 8)
  r = r + __uint_as_float(xor1_u32(__float_as_uint(r)));
  r = r + __uint_as_float(xor2_u32(__float_as_uint(r)));
  return r + __uint_as_float(mirror8_u32(__float_as_uint(r)));
}

}  // namespace cachalot
