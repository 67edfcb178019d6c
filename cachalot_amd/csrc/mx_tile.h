// GEMV tiles on the gfx950 block-scaled matrix cores:
// v_mfma_scale_f32_16x16x128_f8f6f4 with A = fp8 (OCP E4M3) activations and
// B = fp4 (E2M1) weight codes, each 32-element K block of each row / column
// carrying its own E8M0 scale.  One instruction consumes 16 weight rows x 128
// codes -- four times the weights of a bf16 16x16x32 step -- and the weight
// operand needs no conversion to bf16.
//
// Operand layout (lane = 16 * kg + c, c = row of A / column of B):
//   B (fp4, 4 VGPRs): lane (col c, kg) holds K [32 kg, 32 kg + 32), nibble n
//     (byte n / 2, low nibble first) = K 32 kg + n.
//   A (fp8, 8 VGPRs): lane (row c, kg) holds K [16 kg, 16 kg + 16) in bytes
//     0..15 and K [64 + 16 kg, 64 + 16 kg + 16) in bytes 16..31.
//   Scales: the scale of row r (col c) for K block m = K [32 m, 32 m + 32)
//     is the byte `opsel` of the scale operand of lane (r, m) (lane (c, m)).
//   D: D[i][j] sits in lane j + 16 (i / 4), register i % 4.
//
// Activations as fp8 planes.  A bf16 value has an 8-bit significand and an
// E4M3 value a 4-bit one, so a 16-element piece of activations is carried as
// two planes: hi = RNE_e4m3(v / S) and lo = RNE_e4m3(16 (v / S - hi)) with
// S = 2^(E - 7), E the exponent of the piece's largest magnitude, and row
// scales S (hi) and S / 16 (lo).  Every element within 2^13 of the piece's
// largest magnitude is carried exactly (hi + lo / 16 == v / S); smaller ones
// carry an absolute error below 2^-21 of that magnitude.  With weight codes
// exact in E2M1 every product is exact and the instruction accumulates fp32.
//
// Group-separated dot products (2-bit affine banks).  The affine formula
// s * sum(x q) + b * sum(x) needs one dot product per 128-code group.  In a
// step, lane group kg of B carries group 4 b + kg of its weight row (32 codes
// of it per step, four steps per group), and A row r = 4 kg' + 2 h + p carries
// plane p of piece h (16 codes) of the step's 32 codes of group 4 b + kg' and
// zeros elsewhere; its data sits in lane (r, 2 (kg' & 1) + h), in bytes 0..15
// for kg' < 2 and 16..31 for kg' >= 2, and its scale in lane (r, kg').  So the
// four D registers of lane (j, kg) are the four (piece, plane) partial sums of
// group 4 b + kg for weight row j: their sum is the group's exact sum(x q),
// held by the lane that also holds that group's scale and bias.
//
// Plane block: activations are stored per 128-element group.  Piece p (16
// elements) is step c = p / 2, half h = p % 2 of the group's four 32-element steps.
//   [0, 256)   data: [h][plane (hi, lo)][c][16 bytes], the 16 elements of a piece
//              in the order 0, 2, 4, .., 14, 1, 3, .., 15 (the nibble order of
//              q2_spread below), so one lane's four steps are 64 contiguous bytes
//   [256, 272) scales: [h][plane][c] E8M0 bytes, so one u32 holds a lane's four
//              step scales (selected per step by the instruction's opsel)
//   [288, 320) sums: one fp32 per piece, the sum of its 16 values
#pragma once

#include "common.h"

namespace cachalot {
namespace mx {

typedef __attribute__((ext_vector_type(8))) int i32x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int PIECE = 16;
constexpr int GROUP = 128;
constexpr int PIECES = GROUP / PIECE;
constexpr int PB_SCALE = 256;
constexpr int PB_SUM = 288;
constexpr int PB_BYTES = 320;

// Byte offsets of piece p's plane data and scale inside its plane block.
__host__ __device__ inline int pb_data(int p, int plane) { return (((p & 1) * 2 + plane) * 4 + (p >> 1)) * 16; }
__host__ __device__ inline int pb_scale(int p, int plane) { return PB_SCALE + ((p & 1) * 2 + plane) * 4 + (p >> 1); }
constexpr uint32_t E8M0_TWO = 128u;     // 2^1

// D += A (fp8, row scales = byte OPSEL_A of sa) x B (fp4, column scales = byte 0 of sb).
//
// The destination must not share registers with A or B.  This toolchain allows a
// 4-register MFMA destination to overlap its sources, and for this multi-pass
// instruction that corrupted results (data-dependent wrong values and NaNs that
// moved with register allocation).  The empty asm consumes A, B and the result,
// so A and B are live when the result is defined and cannot be reused for it,
// and it keeps the result in AGPRs, a register file A and B are never in.
template <int OPSEL_A = 0, bool ACC_VGPR = false>
__device__ __forceinline__ f32x4_t mfma_fp8_fp4(const i32x8_t& a, const i32x8_t& b, f32x4_t c, uint32_t sa,
                                                uint32_t sb) {
  typedef __attribute__((ext_vector_type(4))) int i32x4_t;
  f32x4_t d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, OPSEL_A, (int)sa, 0, (int)sb);
  const i32x4_t b4 = __builtin_shufflevector(b, b, 0, 1, 2, 3);   // an fp4 B operand is 4 registers
  // the accumulator stays in the AGPRs the instruction writes (pinning it to VGPRs
  // makes the compiler copy it out and back around every instruction); A and B sit
  // in VGPRs, so they cannot overlap it
  // (ACC_VGPR: a kernel whose register budget has no room for AGPR accumulators keeps
  // them in VGPRs)
  if constexpr (ACC_VGPR) asm volatile("" : "+v"(d) : "v"(a), "v"(b4));
  else asm volatile("" : "+a"(d) : "v"(a), "v"(b4));
  return d;
}

// A zero accumulator held in registers (not folded into an inline-constant srcC).
template <bool ACC_VGPR = false>
__device__ __forceinline__ f32x4_t zero_acc() {
  f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (ACC_VGPR) asm volatile("" : "+v"(z));
  else asm volatile("" : "+a"(z));
  return z;
}

// B operand from two u32 words of 2-bit codes (32 codes, low field first): the
// codes are spread into nibbles, code q becoming the E2M1 encoding of q / 2
// (exact with column scale 2).  Nibble n carries code 2n (n < 8), 2(n-8)+1
// (n < 16), then the same pattern +16 for the second word.
__device__ __forceinline__ i32x8_t q2_spread(uint32_t w0, uint32_t w1) {
  i32x8_t b;
  b[0] = (int)(w0 & 0x33333333u);
  b[1] = (int)((w0 >> 2) & 0x33333333u);
  b[2] = (int)(w1 & 0x33333333u);
  b[3] = (int)((w1 >> 2) & 0x33333333u);
  b[4] = 0;
  b[5] = 0;
  b[6] = 0;
  b[7] = 0;
  return b;
}

// Eight 3-bit codes (a 24-bit run, code i at bits 3i) one per nibble, nibble i = code i.
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
  const uint32_t a = (v & 0xFFFu) | ((v << 4) & 0x0FFF0000u);       // four codes per 16-bit half
  const uint32_t b = (a & 0x003F003Fu) | ((a << 2) & 0x3F003F00u);   // two per byte
  return (b & 0x07070707u) | ((b << 1) & 0x70707070u);               // one per nibble
}

// Eight nibble codes (nibble i = code i) one per byte, in order: bytes 0..3 of lo =
// codes 0..3, of hi = codes 4..7.
__device__ __forceinline__ void nibbles_to_bytes(uint32_t n, uint32_t& lo, uint32_t& hi) {
  const uint32_t e = n & 0x0F0F0F0Fu;          // codes 0, 2, 4, 6
  const uint32_t o = (n >> 4) & 0x0F0F0F0Fu;   // codes 1, 3, 5, 7
  lo = __builtin_amdgcn_perm(o, e, 0x05010400u);
  hi = __builtin_amdgcn_perm(o, e, 0x07030602u);
}

// Byte position of element i (0..15) of a piece in its plane.
__device__ __forceinline__ int piece_pos(int i) { return (i & 1) ? 8 + (i >> 1) : (i >> 1); }

__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xffu;
}
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) { return __builtin_amdgcn_cvt_f32_fp8((int)b, 0); }

// Max |v| over each aligned row of 16 lanes (every lane of the row gets it).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __uint_as_float(xor1_u32(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor2_u32(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(mirror8_u32(__float_as_uint(v))));
  return fmaxf(v, __uint_as_float(mirror16_u32(__float_as_uint(v))));
}

struct PieceCode {
  uint32_t hi, lo;      // this lane's element in each plane (E4M3 byte)
  uint32_t scales;      // hi E8M0 | lo E8M0 << 8 (same in every lane of the row)
  float sum;            // sum of the row's 16 values (same in every lane)
};

// Encode the 16 values held by a row of 16 lanes (lane i of the row holds element i;
// every value must be a bf16 number).
__device__ __forceinline__ PieceCode encode_piece(float v) {
  const float m = row16_max(fabsf(v));
  int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;   // zero / subnormal max: -127
  int E = e - 7;
  E = E < -123 ? -123 : (E > 120 ? 120 : E);
  const float inv = __uint_as_float((uint32_t)(127 - E) << 23);   // 2^-E, exact
  const float s = v * inv;
  PieceCode pc;
  pc.hi = f32_to_e4m3(s);
  const float r = s - e4m3_to_f32(pc.hi);                      // exact
  pc.lo = f32_to_e4m3(r * 16.0f);
  pc.scales = (uint32_t)(E + 127) | ((uint32_t)(E + 123) << 8);
  pc.sum = row16_sum(v);
  return pc;
}

// The same encoding with a piece spread over an aligned quad of lanes, 4 elements
// each: lane s of the quad holds elements 4s .. 4s+3.  Returns, per plane, the two
// byte pairs this lane writes: bytes (2s, 2s+1) = elements (4s, 4s+2) and bytes
// (8+2s, 9+2s) = elements (4s+1, 4s+3) (the piece_pos order).
struct PieceCode4 {
  uint32_t hi_a, hi_b, lo_a, lo_b;   // 16-bit pairs for bytes 2s and 8+2s
  uint32_t scales;
  float sum;
};
__device__ __forceinline__ PieceCode4 encode_piece4(float v0, float v1, float v2, float v3) {
  float m = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
  m = fmaxf(m, __uint_as_float(xor1_u32(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(xor2_u32(__float_as_uint(m))));
  int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;
  int E = e - 7;
  E = E < -123 ? -123 : (E > 120 ? 120 : E);
  const float inv = __uint_as_float((uint32_t)(127 - E) << 23);
  const float s0 = v0 * inv, s1 = v1 * inv, s2 = v2 * inv, s3 = v3 * inv;
  PieceCode4 pc;
  pc.hi_a = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s0, s2, 0, false) & 0xffffu;
  pc.hi_b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s1, s3, 0, false) & 0xffffu;
  const float2_t ha = __builtin_amdgcn_cvt_pk_f32_fp8((int)pc.hi_a, false);
  const float2_t hb = __builtin_amdgcn_cvt_pk_f32_fp8((int)pc.hi_b, false);
  pc.lo_a = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32((s0 - ha[0]) * 16.0f, (s2 - ha[1]) * 16.0f, 0, false) & 0xffffu;
  pc.lo_b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32((s1 - hb[0]) * 16.0f, (s3 - hb[1]) * 16.0f, 0, false) & 0xffffu;
  pc.scales = (uint32_t)(E + 127) | ((uint32_t)(E + 123) << 8);
  float sum = (v0 + v1) + (v2 + v3);
  sum = sum + __uint_as_float(xor1_u32(__float_as_uint(sum)));
  pc.sum = sum + __uint_as_float(xor2_u32(__float_as_uint(sum)));
  return pc;
}

__device__ __forceinline__ uint4 lds16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint32_t lds32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Per-lane roles in the group-separated layout (mx_tile.h): which half of the A
// operand carries this lane's data (lo: bytes 0..15, hi: 16..31, or neither) and
// whether it supplies its row's scale.
struct ARole {
  int kgR, halfR, planeR;
  bool lo, hi, scale;
};
__device__ __forceinline__ ARole a_role(int lane) {
  ARole r;
  const int row = lane & 15, kgA = lane >> 4;
  r.kgR = row >> 2;
  r.halfR = (row >> 1) & 1;
  r.planeR = row & 1;
  const bool act = kgA == 2 * (r.kgR & 1) + r.halfR;
  r.lo = act && r.kgR < 2;
  r.hi = act && r.kgR >= 2;
  r.scale = kgA == r.kgR;
  return r;
}

// The A operands of one group-separated chain (four steps) in persistent
// registers: a lane's role never changes, so only its data half is rewritten, by
// one exec-masked block of four contiguous 16-byte LDS reads (the plane block keeps
// a lane's four steps together); the other half, the other lanes' data and the
// other lanes' scales (1.0: their blocks of the row hold zeros, so any finite scale
// gives exact zeros) keep the values set once by chain_init.  The scale lanes read
// one u32 holding their four step scales (byte c for step c).
struct Chain {
  i32x8_t a[4];
  uint32_t sa;
};
__device__ __forceinline__ void chain_init(Chain& ch) {
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) ch.a[c][i] = 0;
  ch.sa = 0x7F7F7F7Fu;
}
__device__ __forceinline__ void chain_load(Chain& ch, const uint8_t* blk, const ARole& ro) {
  const uint8_t* src = blk + (ro.halfR * 2 + ro.planeR) * 64;
  if (ro.lo) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 d = lds16(src + 16 * c);
      ch.a[c][0] = (int)d.x; ch.a[c][1] = (int)d.y; ch.a[c][2] = (int)d.z; ch.a[c][3] = (int)d.w;
    }
  }
  if (ro.hi) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 d = lds16(src + 16 * c);
      ch.a[c][4] = (int)d.x; ch.a[c][5] = (int)d.y; ch.a[c][6] = (int)d.z; ch.a[c][7] = (int)d.w;
    }
  }
  if (ro.scale) ch.sa = lds32(blk + PB_SCALE + (ro.halfR * 2 + ro.planeR) * 4);
}

// mfma_fp8_fp4 with the A scale byte chosen by a step index (a constant once the
// caller's step loop is unrolled).
__device__ __forceinline__ f32x4_t mfma_fp8_fp4_sel(int step, const i32x8_t& a, const i32x8_t& b, f32x4_t c,
                                                    uint32_t sa, uint32_t sb) {
  switch (step & 3) {
    case 0: return mfma_fp8_fp4<0>(a, b, c, sa, sb);
    case 1: return mfma_fp8_fp4<1>(a, b, c, sa, sb);
    case 2: return mfma_fp8_fp4<2>(a, b, c, sa, sb);
    default: return mfma_fp8_fp4<3>(a, b, c, sa, sb);
  }
}

// One step of a chain into a single persistent operand `a` (set up like a chain's
// registers: zeros, written once): only the lane's data half is rewritten, from
// chunk c's 16 bytes of the plane block.  The step scales come from chain_scales.
__device__ __forceinline__ void chain_load_step(i32x8_t& a, const uint8_t* blk, const ARole& ro, int c) {
  const uint8_t* src = blk + (ro.halfR * 2 + ro.planeR) * 64 + 16 * c;
  if (ro.lo) {
    const uint4 d = lds16(src);
    a[0] = (int)d.x; a[1] = (int)d.y; a[2] = (int)d.z; a[3] = (int)d.w;
  }
  if (ro.hi) {
    const uint4 d = lds16(src);
    a[4] = (int)d.x; a[5] = (int)d.y; a[6] = (int)d.z; a[7] = (int)d.w;
  }
}
// The scale lanes' four chunk scales of a plane block (byte c for chunk c).
__device__ __forceinline__ void chain_scales(uint32_t& sa, const uint8_t* blk, const ARole& ro) {
  if (ro.scale) sa = lds32(blk + PB_SCALE + (ro.halfR * 2 + ro.planeR) * 4);
}

__device__ __forceinline__ float dot4(const f32x4_t& d) { return (d[0] + d[1]) + (d[2] + d[3]); }

// Sum of the first `npieces` piece sums of a plane block (fixed order).
__device__ __forceinline__ float piece_sums(const uint8_t* blk, int npieces) {
  const float4 a = *reinterpret_cast<const float4*>(blk + PB_SUM);
  const float4 b = *reinterpret_cast<const float4*>(blk + PB_SUM + 16);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float s = 0.0f;
#pragma unroll
  for (int p = 0; p < PIECES; ++p) s = s + (p < npieces ? v[p] : 0.0f);
  return s;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return bf16_to_f32((uint16_t)w); }

// Encode one quad of x (4 bf16, t4 = quad index: elements 4 t4 .. 4 t4 + 3) into the
// plane blocks at `planes` (one per 128 elements).  The four lanes of an aligned
// lane quad must encode the four quads of one piece together.
__device__ __forceinline__ void encode_x_quad(uint8_t* planes, int t4, uint2 xv) {
  const float v0 = bf16_to_f32((uint16_t)xv.x), v1 = bf16_to_f32((uint16_t)(xv.x >> 16));
  const float v2 = bf16_to_f32((uint16_t)xv.y), v3 = bf16_to_f32((uint16_t)(xv.y >> 16));
  const PieceCode4 pc = encode_piece4(v0, v1, v2, v3);
  const int P = t4 >> 2, q4 = t4 & 3, pp = P & 7;
  uint8_t* gb = planes + (P >> 3) * PB_BYTES;
  uint8_t* hi = gb + pb_data(pp, 0);
  uint8_t* lo = gb + pb_data(pp, 1);
  *reinterpret_cast<uint16_t*>(hi + 2 * q4) = (uint16_t)pc.hi_a;
  *reinterpret_cast<uint16_t*>(hi + 8 + 2 * q4) = (uint16_t)pc.hi_b;
  *reinterpret_cast<uint16_t*>(lo + 2 * q4) = (uint16_t)pc.lo_a;
  *reinterpret_cast<uint16_t*>(lo + 8 + 2 * q4) = (uint16_t)pc.lo_b;
  if (q4 == 0) {
    gb[pb_scale(pp, 0)] = (uint8_t)pc.scales;
    gb[pb_scale(pp, 1)] = (uint8_t)(pc.scales >> 8);
    *reinterpret_cast<float*>(gb + PB_SUM + 4 * pp) = pc.sum;
  }
}

}  // namespace mx
}  // namespace cachalot
