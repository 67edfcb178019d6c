// Shared pieces of the block-scaled prefill kernels (prefill_mx.hip: FP4, 2-bit g128
// and affine groups of 128 on 16 x 16 x 128 instructions; prefill_affine_mx.hip:
// affine groups of 64 on 32 x 32 x 64 instructions): tile constants, weight kinds,
// the kernel arguments and the code-to-operand conversions.
#pragma once

#include "decode_common.h"
#include "mfma_tile.h"
#include "mx_tile.h"

namespace cachalot {
namespace pmx {

using namespace decode;

constexpr int P3_THREADS = 256;
constexpr int P3_WAVES = 4;
constexpr int P3_MT = 64;                     // token rows per tile
constexpr int P3_TB = P3_MT / 16;             // token fragments
constexpr int P3_STAGES = 2;
constexpr int P3_ROWB = 256;                  // one row's chunk: hi 128 B | lo 128 B
constexpr int P3_ABYTES = P3_MT * P3_ROWB;    // 16 KiB per stage
constexpr int P3_ASLOTS = P3_ABYTES / 16 / P3_THREADS;   // 16-byte A slots per lane and chunk (4)

typedef __attribute__((ext_vector_type(8))) int i32x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// Weight kinds of p3_kernel (AK): FP4; 2-bit g128 with the codes as fp4 operands;
// (BITS << 8) | G for affine codes as fp8 operands (code q as the E4M3 byte q, which
// is q * 2^-9 -- subnormal below 8 -- with B scale 2^9).
constexpr int AK_FP4 = 0;
constexpr int AK_Q2 = 1;
constexpr int ak_aff(int bits, int g) { return (bits << 8) | g; }
constexpr bool ak_fold(int ak) { return ak != AK_FP4; }       // group formula per group
constexpr bool ak_bytes(int ak) { return ak > AK_Q2; }        // codes as fp8 bytes
constexpr int ak_bits(int ak) { return ak == AK_Q2 ? 2 : ak >> 8; }
constexpr int ak_group(int ak) { return ak <= AK_Q2 ? 128 : (ak & 255); }
constexpr int ak_gpc(int ak) { return ak_fold(ak) ? 128 / ak_group(ak) : 1; }   // groups per K chunk
constexpr uint32_t E8M0_2P9 = 136u;                            // 2^9

struct MxArgs {
  const uint8_t* ap;          // A planes [source rows][kch][256]
  const uint8_t* as;          // A scales [source rows][sb]
  int sb;                     // A scale bytes per source row
  int kch;                    // 128-element chunks along K (K_pad / 128)
  const int32_t* a_gather;    // source row of a tile row (row_token) or null (the row itself)
  const uint8_t* pool;
  Layout L;
  const int32_t* slot_table;
  const int32_t* offsets;
  const int2* tiles;
  const int32_t* tiles_n;
  const int32_t* row_token;
  const int32_t* row_slot;
  const float* row_w;
  int K;                      // real K (D or F)
  int N;                      // weight rows per matrix (F or D)
  int k;
  float limit;
  uint8_t* hp;                // gate/up: h planes [rows][hkch][256]
  uint8_t* hs;                // gate/up: h scales [rows][hsb]
  int hsb, hkch;
  uint16_t* y;                // down: [T, k, N]
  const float* asum;          // 2-bit: chunk sums of the A source rows [source rows][kch]
  float* hsum;                // 2-bit gate/up: chunk sums of h [rows][hkch]
};

__host__ __device__ inline int scale_row_bytes(int K) { return (K / 32 * 2 + 15) / 16 * 16; }

// Plane scale exponent of a block whose largest magnitude is m: E = e(m) - 7,
// clamped so that both E8M0 bytes (E + 127, E + 123) are finite scales.
__device__ __forceinline__ int plane_exp(float m) {
  const int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;   // zero / subnormal max: -127
  const int E = e - 7;
  return E < -123 ? -123 : (E > 120 ? 120 : E);
}

// Sixteen 2-bit codes (the low or high half of a word) one per nibble in natural
// order, nibble n = E2M1 of code n / 2.
__device__ __forceinline__ uint32_t q2_nibbles(uint32_t v16) {
  uint32_t t = (v16 & 0xFFu) | ((v16 & 0xFF00u) << 8);
  t = (t & 0x000F000Fu) | ((t & 0x00F000F0u) << 4);
  return (t & 0x03030303u) | ((t & 0x0C0C0C0Cu) << 2);
}

// The fp8 B operand of a lane from its two code runs (one code per byte).
template <int BITS>
__device__ __forceinline__ i32x8_t aff_code_bytes(const uint4& w, int kg) {
  uint32_t o[8];
  if constexpr (BITS == 4) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) mx::nibbles_to_bytes(v[j], o[2 * j], o[2 * j + 1]);
  } else if constexpr (BITS == 2) {
    const uint32_t v[2] = {w.x, w.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      mx::nibbles_to_bytes(q2_nibbles(v[j] & 0xFFFFu), o[4 * j], o[4 * j + 1]);
      mx::nibbles_to_bytes(q2_nibbles(v[j] >> 16), o[4 * j + 2], o[4 * j + 3]);
    }
  } else {
    const uint32_t sh = (uint32_t)(2 * BITS * kg & 3) * 8;   // the run's offset in its first word
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t lo = __builtin_amdgcn_alignbit(v[2 * j + 1], v[2 * j], sh);
      const uint32_t hi = v[2 * j + 1] >> sh;
      mx::nibbles_to_bytes(mx::spread3(lo & 0xFFFFFFu), o[4 * j], o[4 * j + 1]);
      mx::nibbles_to_bytes(mx::spread3(__builtin_amdgcn_alignbit(hi, lo, 24) & 0xFFFFFFu), o[4 * j + 2],
                           o[4 * j + 3]);
    }
  }
  return i32x8_t{(int)o[0], (int)o[1], (int)o[2], (int)o[3], (int)o[4], (int)o[5], (int)o[6], (int)o[7]};
}

}  // namespace pmx
}  // namespace cachalot
