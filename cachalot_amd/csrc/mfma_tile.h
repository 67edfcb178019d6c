// Expert-GEMV tiles on the bf16 matrix cores of gfx950
// (v_mfma_f32_16x16x32_bf16, D = A x B + C, fp32 accumulation).
//
// Operand layout of that instruction (64 lanes, lane = 16 * kg + c):
//   A (16 x 32): lane (row c, k-group kg) holds A[c][8kg .. 8kg+7] as 8 bf16;
//   B (32 x 16): lane (col c, k-group kg) holds B[8kg .. 8kg+7][c];
//   D (16 x 16): D[i][j] sits in lane j + 16 * (i / 4), register i % 4.
//
// A decode tile is 16 weight rows (the B columns, lane & 15) by 32 codes per
// step: lane group kg (= lane >> 4) walks its own run of quantisation groups
// 8 codes per step.  The activation vector is the A operand and lives in LDS:
// the lanes that carry it read their 16 bytes per step, every other lane reads
// a zero region, so one step costs one ds_read_b128 per wave however many
// weight matrices share it.  Which A rows carry data decides what the D rows
// hold:
//   * 2-bit banks: lane (row 4kg, kg) carries the activations of lane group
//     kg's group, so D[4kg][j] -- lane j + 16kg, register 0 -- is exactly that
//     group's sum(x q) for weight row j, and the lane that loaded the group's
//     scale and bias applies MLX's group formula s * sum(x q) + b * sum(x).
//   * FP4 banks: the E8M0 scale is applied by the converter, so every lane
//     carries the activations (row c of A = x for all c) and D[0][j] is the
//     plain dot product; an fp32 hidden vector is split into bf16 hi + lo
//     parts carried by A rows 0 and 1 (D[0][j] + D[1][j]).
//
// 2-bit codes become bf16 through the FP4 converter: the codes of a u32 word
// are spread into nibbles (code q is the E2M1 encoding of q / 2) and converted
// with scale 2.  Converter byte b of ev = w & 0x33333333 holds codes (4b, 4b+2),
// of od = (w >> 2) & 0x33333333 codes (4b+1, 4b+3), so the 8 codes of half H of
// a word arrive in the order 0, 2, 1, 3, 4, 6, 5, 7 ("MFMA order"), and the
// activations are stored in LDS in that same order.  Products of bf16
// activations with small integers or with E2M1 x 2^e values are exact.
#pragma once

#include "common.h"

namespace cachalot {
namespace tile {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int GROUP = 128;               // 2-bit quantisation group (codes)
constexpr int LDS_GROUP_BYTES = 272;     // 128 bf16 + 16 bytes of padding (bank spread)
constexpr int LDS_ZERO_BYTES = 256;      // 16 steps x 16 bytes of zeros

__device__ __forceinline__ f32x4_t mfma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t lds_a(const uint8_t* base, uint32_t off) {
  return *reinterpret_cast<const bf16x8_t*>(base + off);
}

// Position of value t (0..7) of an 8-value piece in MFMA order.
__device__ __forceinline__ int mfma8_pos(int t) { return (t & 4) | ((t & 1) << 1) | ((t >> 1) & 1); }

// Element n of a vector stored group-major in MFMA order.
__device__ __forceinline__ int mfma_index(int n) { return (n & ~7) | mfma8_pos(n & 7); }

// B operand of step half H from one u32 word of 16 2-bit codes (values 0..3 as bf16).
template <int H>
__device__ __forceinline__ bf16x8_t q2_codes_to_b(uint32_t w) {
  const uint32_t ev = w & 0x33333333u;
  const uint32_t od = (w >> 2) & 0x33333333u;
  uint32_t p[4];
  p[0] = fp4x2_to_bf16x2<2 * H>(ev, 2.0f);
  p[1] = fp4x2_to_bf16x2<2 * H>(od, 2.0f);
  p[2] = fp4x2_to_bf16x2<2 * H + 1>(ev, 2.0f);
  p[3] = fp4x2_to_bf16x2<2 * H + 1>(od, 2.0f);
  return __builtin_bit_cast(bf16x8_t, p);
}

// B operand from one u32 word of 8 FP4 nibbles (natural order, low nibble first),
// each value times `scale` (an E8M0 power of two): exact bf16.
__device__ __forceinline__ bf16x8_t fp4_codes_to_b(uint32_t w, float scale) {
  uint32_t p[4];
  p[0] = fp4x2_to_bf16x2<0>(w, scale);
  p[1] = fp4x2_to_bf16x2<1>(w, scale);
  p[2] = fp4x2_to_bf16x2<2>(w, scale);
  p[3] = fp4x2_to_bf16x2<3>(w, scale);
  return __builtin_bit_cast(bf16x8_t, p);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// (v0,v1),(v2,v3) -> (v0,v2),(v1,v3)
__device__ __forceinline__ void pairs_mfma(uint32_t a, uint32_t b, uint32_t& e, uint32_t& o) {
  e = (a & 0xffffu) | (b << 16);
  o = (a >> 16) | (b & 0xffff0000u);
}

constexpr uint32_t BF16_ONES = 0x3f803f80u;

__device__ __forceinline__ float sum_bf16x8(uint4 v) {
  float s = 0.0f;
  s = dot2_bf16(v.x, BF16_ONES, s);
  s = dot2_bf16(v.y, BF16_ONES, s);
  s = dot2_bf16(v.z, BF16_ONES, s);
  s = dot2_bf16(v.w, BF16_ONES, s);
  return s;
}

// Sum over each aligned group of 8 lanes (all 8 lanes end with the same value).
__device__ __forceinline__ float sum8_lanes(float v) {
  v = v + __uint_as_float(xor1_u32(__float_as_uint(v)));
  v = v + __uint_as_float(xor2_u32(__float_as_uint(v)));
  return v + __uint_as_float(mirror8_u32(__float_as_uint(v)));
}

// Sum over the four lane groups (lanes j, j+16, j+32, j+48).
__device__ __forceinline__ float sum_lane_groups(float v) {
  v = v + xor_f<16>(v);
  return v + xor_f<32>(v);
}

// Copy `bytes` (a multiple of 16) from global memory straight into LDS with the
// gfx950 direct-to-LDS load (global_load_lds_dwordx4: lane l of a wave writes
// dst + 16 l), wave-cooperatively: wave w of nwaves copies the 1 KiB chunks w,
// w + nwaves, ...  No registers are involved; the copy is complete once the
// wave's vector-memory counter has drained (wait_vmem) and, for other waves'
// chunks, after the following workgroup barrier.  COHERENT = 1 reads at agent
// scope (sc1), for data other workgroups of the same launch published with
// agent-coherent stores.
template <int COHERENT = 0>
__device__ __forceinline__ void dma_to_lds(const void* src, uint8_t* dst, int bytes, int wave, int nwaves,
                                           int lane) {
  for (int c = wave * 1024; c < bytes; c += nwaves * 1024) {
    const int off = c + lane * 16;
    if (off < bytes)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(src) + off, dst + c, 16, 0,
                                       COHERENT ? 16 : 0);
  }
}

// One direct-to-LDS load of 16 bytes per lane (lane l writes lds + 16 l), issued as
// inline asm so the compiler's wait-count tracking does not see it: that tracking
// cannot tell which LDS reads depend on which such load and would otherwise wait for
// every outstanding load before the first LDS read.  The caller guarantees
// completion: a later wait for a register load issued after this one (loads
// complete in issue order), or wait_vmem().  Clobbers m0.
__device__ __forceinline__ void lds_load16_untracked(const void* src, void* lds) {
  const uint32_t la = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(la), "v"(src) : "memory", "m0");
}

// Copy `bytes` (a multiple of 16) into LDS with untracked direct-to-LDS loads: 1 KiB
// chunks c = part, part + parts, ...  The caller waits (wait_vmem, or a wait count
// for register loads issued later) before the data is read.
__device__ __forceinline__ void copy_to_lds_untracked(const uint8_t* src, uint8_t* dst, int bytes, int part,
                                                      int parts, int lane) {
  for (int c = part * 1024; c < bytes; c += parts * 1024)
    if (c + 16 * lane < bytes) lds_load16_untracked(src + c + 16 * lane, dst + c);
}

// s_waitcnt immediate (gfx9 encoding) for "at most n vector-memory loads of this wave
// still outstanding", expcnt and lgkmcnt unconstrained; n < 64.
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// Wait until every vector-memory load of this wave has landed (registers and LDS).
// (The builtin, unlike inline asm, is visible to the compiler's wait-count tracking, so
// it knows that LDS written by direct-to-LDS loads is complete after it.)
__device__ __forceinline__ void wait_vmem() {
  __builtin_amdgcn_s_waitcnt(0x0F70);   // gfx9 encoding: vmcnt(0), expcnt and lgkmcnt unconstrained
  asm volatile("" ::: "memory");
}

}  // namespace tile
}  // namespace cachalot
