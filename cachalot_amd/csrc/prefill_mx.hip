// FP4 prefill (expert-major grouped GEMM) on the gfx950 block-scaled matrix cores.
//
// Reference: routed_expert_forward_sgmm / routed_expert_forward_batched
// (src/cachalot/model/fp4_sgmm_metal.py:257-333, moe_prefill_batched.py:31-61),
// called per expert from moe_prefill_grouped.py:420-467.  Rounding points:
// g = bf16(x W1), u = bf16(x W3), h = bf16(silu(min(g, L)) * clip(u, +-L) * w),
// y = bf16(h W2); the products accumulate in fp32.
//
// v_mfma_scale_f32_16x16x128_f8f6f4 multiplies A = fp8 (OCP E4M3) by B = fp4
// (E2M1), each operand carrying one E8M0 scale per 32-element K block.  The
// bank's FP4 weights are exactly that B operand: the packed codes go in as they
// are stored and their E8M0 block scales are the B scales, so no weight is
// converted.  The activations (x for gate/up, h for down) are bf16 and go in as
// two fp8 planes per 32-element block: with S = 2^(E - 7), E the exponent of the
// block's largest magnitude, hi = RNE_e4m3(v / S) and lo = RNE_e4m3(16 (v / S -
// hi)), scales S and S / 16.  hi + lo / 16 == v / S for every element within
// 2^13 of the block's largest magnitude (bf16 has 8 significant bits, each plane
// 4); smaller elements carry an absolute error below 2^-21 of that magnitude.
// Products of E4M3 and E2M1 values are exact; the instruction accumulates fp32.
//
// Layouts (workspace, written by these kernels):
//   planes  [rows][K_pad / 128][256 B]: per 128-element chunk, hi bytes 0..127
//           then lo bytes 128..255, element order;
//   scales  [rows][sb B]: per 32-element block b, bytes 2b (hi) and 2b + 1 (lo),
//           sb a multiple of 16.
// x_planes_kernel writes x's planes per token; the gate/up kernel's epilogue
// writes h's planes per permuted row (columns past F are zero, so K_pad = F
// rounded up to 128 reads zeros there).
//
// Tiling: one 256-thread workgroup = a 64-row M tile of one expert (rows of the
// expert-major permutation, tile list of grouped.hip) x 16 NF rows per wave of
// each of NM matrices (gate/up: NM = 2, W1 and W3, NF = 2 -> 128 rows of each;
// down: NM = 1, NF = 4 -> 256 rows of W2).  K runs in chunks of 128: the A planes
// of the chunk through a two-stage LDS ring filled by direct-to-LDS loads
// (16-byte slots XOR-swizzled by row, so the operand reads hit distinct banks),
// the wave's codes one chunk ahead in registers, the B scales 32 bytes (eight
// chunks) per lane and load, one trip of eight chunks ahead.  The tile's A scales sit
// in LDS for the whole K loop.  Three workgroups fit a CU (49 KiB of LDS, ~100 VGPRs +
// 64 AGPRs each): measured 3.51 ms per config-3 layer against 3.64 with a three-stage
// ring (two chunks ahead), which left room for two.  Workgroups go to the XCDs
// round-robin by launch index; the mapping gives every slice of one tile to one XCD,
// so the tile's A rows are fetched into that XCD's L2 once.
//
// Affine banks (AK != AK_FP4) run the same kernels with the group formula
// s * sum(x q) + b * sum(x) applied per 128-code group, one group per K chunk: each
// chunk's two plane instructions accumulate into a zeroed tile, folded into fp32
// accumulators in VGPRs as acc = fma(s, tile, fma(b, sum x, acc)) with the weight
// row's scale and bias and the token row's group sum of x (or h).  2-bit g128 codes go
// in as the fp4 operand (E2M1 of q / 2 with B scale 2, spread into natural nibble
// order); 3- and 4-bit g128 codes as fp8 bytes (prefill_mx.h).  The scales and biases
// come eight groups per 16-byte load, each chunk's pair shuffled to the lanes.  The
// group sums come from the plane writers (x_planes_rows_kernel; the gate/up epilogue
// for h, whose workgroup holds one whole 128-column chunk of h).  Groups of 64 run on
// prefill_affine_mx.hip's 32 x 32 x 64 kernels over the same planes.
#include <type_traits>

#include "decode_common.h"
#include "mfma_tile.h"
#include "mx_tile.h"
#include "prefill_mx.h"

namespace cachalot {

// affine groups of 64 (prefill_affine_mx.hip)
int launch_prefill_affine_g64(int ak, const pmx::MxArgs& gu, int s_gu, size_t lds_gu, const pmx::MxArgs& dn,
                              int s_dn, size_t lds_dn, int tiles8, hipStream_t s);

namespace {

using namespace decode;
using namespace pmx;

// D += A (fp8 plane, row scales = byte OPSEL_A of sa) x B (fp4 codes, column scales = byte 0 of sb).
// The destination must not share registers with A or B (see mx_tile.h).  The empty
// asm pins the accumulator to the AGPRs, where the MFMA keeps it (A and B live in
// VGPRs, so they cannot overlap it), and keeps A and B live until the result exists;
// pinning it to VGPRs instead makes the compiler copy it out of and back into AGPRs
// around every instruction.
// B_FP8: B is fp8 (E4M3, all eight registers) instead of fp4 (the first four).
template <int OPSEL_A, bool B_FP8 = false>
__device__ __forceinline__ f32x4_t mfma_plane(const i32x8_t& a, const i32x8_t& b, f32x4_t c, uint32_t sa,
                                              uint32_t sb) {
  typedef __attribute__((ext_vector_type(4))) int i32x4_t;
  f32x4_t d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, B_FP8 ? 0 : 4, OPSEL_A, (int)sa, 0,
                                                                (int)sb);
  if constexpr (B_FP8) {
    asm volatile("" : "+a"(d) : "v"(a), "v"(b));
  } else {
    const i32x4_t b4 = __builtin_shufflevector(b, b, 0, 1, 2, 3);
    asm volatile("" : "+a"(d) : "v"(a), "v"(b4));
  }
  return d;
}

// Two fp8 planes of 8 values: hi = RNE(v * inv), lo = RNE(16 (v * inv - hi)).
__device__ __forceinline__ void encode8(const float (&v)[8], float inv, uint2& hi, uint2& lo) {
  float s[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = v[j] * inv;   // exact: inv is a power of two
  uint32_t h0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[0], s[1], 0, false);
  h0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[2], s[3], (int)h0, true);
  uint32_t h1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[4], s[5], 0, false);
  h1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[6], s[7], (int)h1, true);
  float2_t p[4];
  p[0] = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, false);
  p[1] = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, true);
  p[2] = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, false);
  p[3] = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, true);
  float r[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[2 * j] = (s[2 * j] - p[j][0]) * 16.0f;       // exact
    r[2 * j + 1] = (s[2 * j + 1] - p[j][1]) * 16.0f;
  }
  uint32_t l0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
  l0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], (int)l0, true);
  uint32_t l1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r[4], r[5], 0, false);
  l1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r[6], r[7], (int)l1, true);
  hi = make_uint2(h0, h1);
  lo = make_uint2(l0, l1);
}

// x [T, D] bf16 -> planes and scales per token.  One thread = 8 values; the four
// threads of an aligned lane quad hold one 32-element block.
__global__ void __launch_bounds__(256) x_planes_rows_kernel(const uint16_t* __restrict__ x, int T, int D,
                                                            uint8_t* __restrict__ xp, uint8_t* __restrict__ xs,
                                                            int sb, float* __restrict__ xsum, int gsum) {
  const int64_t t8 = (int64_t)blockIdx.x * 256 + threadIdx.x;   // index of an 8-value group
  const int per_row = D / 8;
  const bool live = t8 < (int64_t)T * per_row;
  const int64_t tc = live ? t8 : 0;
  const int t = (int)(tc / per_row), g8 = (int)(tc - (int64_t)t * per_row);
  const uint4 raw = *reinterpret_cast<const uint4*>(x + (size_t)t * D + 8 * g8);
  float v[8];
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(w[j] << 16);
    v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  m = fmaxf(m, __uint_as_float(xor1_u32(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(xor2_u32(__float_as_uint(m))));
  const int E = plane_exp(m);
  uint2 hi, lo;
  encode8(v, __uint_as_float((uint32_t)(127 - E) << 23), hi, lo);
  // the group sums of affine banks' group formula (gsum = 128: 16 threads per group,
  // 64: 8 threads)
  float cs = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) cs = cs + v[j];
  cs = cs + __uint_as_float(xor1_u32(__float_as_uint(cs)));
  cs = cs + __uint_as_float(xor2_u32(__float_as_uint(cs)));
  cs = cs + __uint_as_float(mirror8_u32(__float_as_uint(cs)));
  if (gsum == 128) cs = cs + __uint_as_float(mirror16_u32(__float_as_uint(cs)));
  if (!live) return;
  const int tpg = gsum / 8;   // threads per group
  if (xsum != nullptr && g8 % tpg == 0) xsum[(size_t)t * (D / gsum) + g8 / tpg] = cs;
  const int col = 8 * g8, ch = col >> 7, byte = col & 127;
  uint8_t* dst = xp + ((size_t)t * (D / 128) + ch) * P3_ROWB + byte;
  *reinterpret_cast<uint2*>(dst) = hi;
  *reinterpret_cast<uint2*>(dst + 128) = lo;
  if ((g8 & 3) == 0) {
    const uint32_t sc = (uint32_t)(E + 127) | ((uint32_t)(E + 123) << 8);
    *reinterpret_cast<uint16_t*>(xs + (size_t)t * sb + (col / 32) * 2) = (uint16_t)sc;
  }
}

template <int NM, int NF>
struct P3Chunk {
  uint4 codes[NM][NF];
};

template <int NM, int NF>
__device__ __forceinline__ void p3_issue(uint8_t* stage, const uint8_t* (&asrc)[P3_ASLOTS],
                                         const uint8_t* (&wrow)[NM][NF], int c, int kg, int wave, int row_bytes,
                                         P3Chunk<NM, NF>& out) {
#pragma unroll
  for (int q = 0; q < P3_ASLOTS; ++q)
    tile::lds_load16_untracked(asrc[q] + (size_t)c * P3_ROWB, stage + (P3_ASLOTS * wave + q) * 1024);
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f)
      out.codes[m][f] = *reinterpret_cast<const uint4*>(wrow[m][f] + min(c * 64 + kg * 16, row_bytes - 16));
}

// 2-bit: block kg of the chunk's group (32 codes, 8 bytes) per (matrix, fragment);
// rows as 32-bit offsets from the slot record (a uniform base), so no 64-bit address
// per row stays live.  (The groups' scales and biases come eight at a time, p3_kernel.)
template <int NM, int NF>
__device__ __forceinline__ void p3_issue_q2(uint8_t* stage, const uint8_t* (&asrc)[P3_ASLOTS], const uint8_t* base,
                                            const int (&woff)[NM], const int (&nrow)[NF], int c, int kg, int wave,
                                            int row_bytes, P3Chunk<NM, NF>& out) {
#pragma unroll
  for (int q = 0; q < P3_ASLOTS; ++q)
    tile::lds_load16_untracked(asrc[q] + (size_t)c * P3_ROWB, stage + (P3_ASLOTS * wave + q) * 1024);
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint2 v = *reinterpret_cast<const uint2*>(base + woff[m] + nrow[f] * row_bytes + c * 32 + kg * 8);
      out.codes[m][f] = make_uint4(v.x, v.y, 0u, 0u);
    }
}

// B scales of chunk c = 4 g + J from the group registers (lane (i, p) holds the 16
// E8M0 bytes of group g -- chunks 4g .. 4g+3 -- of weight row i of pair p = (m, f)):
// lane (i, kg) takes byte kg of word J from lane (i, p).  Blocks past K: 127.
template <int NM, int NF>
__device__ __forceinline__ void p3_scales(const uint4& grp, int J, int c, int i, int kg, int blocks,
                                          uint32_t (&bs)[NM][NF]) {
  const uint32_t w = J == 0 ? grp.x : J == 1 ? grp.y : J == 2 ? grp.z : grp.w;
  const bool in_k = 4 * c + kg < blocks;
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint32_t v = (uint32_t)__shfl((int)w, 16 * (m * NF + f) + i, 64);
      bs[m][f] = in_k ? (v >> (8 * kg)) & 0xffu : 127u;
    }
}

template <int NM, int NF>
__device__ __forceinline__ void p3_compute(const uint8_t* ab, const uint8_t* sbuf, int sbs, const P3Chunk<NM, NF>& ch,
                                           const uint32_t (&bs)[NM][NF], int c, int i, int kg, int ntb,
                                           f32x4_t (&acc)[NM][NF][P3_TB]) {
  i32x8_t b[NM][NF];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint4 w = ch.codes[m][f];
      b[m][f] = i32x8_t{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
    }
#pragma unroll
  for (int tb = 0; tb < P3_TB; ++tb) {
    if (tb >= ntb) break;
    const int row = tb * 16 + i;
    const uint8_t* ar = ab + row * P3_ROWB;
    const uint4 h0 = mx::lds16(ar + ((kg ^ i) << 4));
    const uint4 h1 = mx::lds16(ar + (((4 + kg) ^ i) << 4));
    const uint4 l0 = mx::lds16(ar + (((8 + kg) ^ i) << 4));
    const uint4 l1 = mx::lds16(ar + (((12 + kg) ^ i) << 4));
    const uint32_t sa = *reinterpret_cast<const uint16_t*>(sbuf + row * sbs + (4 * c + kg) * 2);
    const i32x8_t ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
    const i32x8_t alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) acc[m][f][tb] = mfma_plane<0>(ahi, b[m][f], acc[m][f][tb], sa, bs[m][f]);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) acc[m][f][tb] = mfma_plane<1>(alo, b[m][f], acc[m][f][tb], sa, bs[m][f]);
  }
}

// 2-bit chunk: per token block, the two plane instructions of every (matrix, fragment)
// into zeroed tiles, then the group formula folded into the fp32 accumulators.
template <int NM, int NF>
__device__ __forceinline__ void p3_compute_q2(const uint8_t* ab, const uint8_t* sbuf, int sbs, const float* sxs,
                                              const P3Chunk<NM, NF>& ch, const uint32_t (&sbw)[NM][NF], int c, int i,
                                              int kg, int ntb, bool f16, float (&acc)[NM][NF][P3_TB][4]) {
  i32x8_t b[NM][NF];
  float sc[NM][NF], bi[NM][NF];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint4 w = ch.codes[m][f];
      b[m][f] = i32x8_t{(int)q2_nibbles(w.x & 0xFFFFu), (int)q2_nibbles(w.x >> 16), (int)q2_nibbles(w.y & 0xFFFFu),
                        (int)q2_nibbles(w.y >> 16), 0, 0, 0, 0};
      sc[m][f] = scale_bits_to_f32((uint16_t)(sbw[m][f] & 0xFFFFu), f16);
      bi[m][f] = scale_bits_to_f32((uint16_t)(sbw[m][f] >> 16), f16);
    }
#pragma unroll
  for (int tb = 0; tb < P3_TB; ++tb) {
    if (tb >= ntb) break;
    const int row = tb * 16 + i;
    const uint8_t* ar = ab + row * P3_ROWB;
    const uint4 h0 = mx::lds16(ar + ((kg ^ i) << 4));
    const uint4 h1 = mx::lds16(ar + (((4 + kg) ^ i) << 4));
    const uint4 l0 = mx::lds16(ar + (((8 + kg) ^ i) << 4));
    const uint4 l1 = mx::lds16(ar + (((12 + kg) ^ i) << 4));
    const uint32_t sa = *reinterpret_cast<const uint16_t*>(sbuf + row * sbs + (4 * c + kg) * 2);
    const float4 sx = *reinterpret_cast<const float4*>(sxs + c * P3_MT + tb * 16 + 4 * kg);
    const i32x8_t ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
    const i32x8_t alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
    f32x4_t d[NM][NF];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) d[m][f] = mfma_plane<0>(ahi, b[m][f], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, sa, mx::E8M0_TWO);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) d[m][f] = mfma_plane<1>(alo, b[m][f], d[m][f], sa, mx::E8M0_TWO);
    const float sxv[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[m][f][tb][r] = fmaf(sc[m][f], d[m][f][r], fmaf(bi[m][f], sxv[r], acc[m][f][tb][r]));
  }
}

// Affine codes as fp8 operands.  Lane group kg of the instruction's fp8 operand holds
// elements 16 kg .. 16 kg + 15 of the chunk (registers 0..3) and 64 + 16 kg .. (4..7),
// the A planes' order; the matching codes are the two runs of 16 codes at those
// elements, 2 BITS bytes each: run 0 at byte 2 BITS kg of the row's chunk, run 1 at
// 8 BITS + 2 BITS kg.  Each run is loaded as whole words (3-bit: the 8 bytes from the
// 4-byte boundary below it) into codes[m][f] (run 0: x / y, run 1: z / w).  Groups
// of 128 only here (one per chunk; the rows hold whole groups); groups of 64 run on
// prefill_affine_mx.hip's kernels.
template <int AK, int NM, int NF>
__device__ __forceinline__ void p3_issue_aff(uint8_t* stage, const uint8_t* (&asrc)[P3_ASLOTS], const uint8_t* base,
                                             const int (&woff)[NM], const int (&nrow)[NF], int c, int kg, int wave,
                                             int row_bytes, P3Chunk<NM, NF>& out) {
  static_assert(ak_group(AK) == 128, "one group per chunk");
  constexpr int BITS = ak_bits(AK), CB = 16 * BITS;
  constexpr int LB = BITS == 2 ? 4 : 8;   // bytes per run load
#pragma unroll
  for (int q = 0; q < P3_ASLOTS; ++q)
    tile::lds_load16_untracked(asrc[q] + (size_t)c * P3_ROWB, stage + (P3_ASLOTS * wave + q) * 1024);
  const int r0 = (2 * BITS * kg) & ~3, r1 = r0 + 8 * BITS;
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint8_t* row = base + woff[m] + nrow[f] * row_bytes;
      const int o0 = min(c * CB + r0, row_bytes - LB), o1 = min(c * CB + r1, row_bytes - LB);
      if constexpr (BITS == 2) {
        out.codes[m][f] = make_uint4(*reinterpret_cast<const uint32_t*>(row + o0),
                                     *reinterpret_cast<const uint32_t*>(row + o1), 0u, 0u);
      } else {
        const uint2 a = *reinterpret_cast<const uint2*>(row + o0);
        const uint2 b = *reinterpret_cast<const uint2*>(row + o1);
        out.codes[m][f] = make_uint4(a.x, a.y, b.x, b.y);
      }
    }
}

// Affine chunk with fp8 codes (groups of 128): per token block, the two plane
// instructions into a zeroed tile, then the group formula folded in.
template <int AK, int NM, int NF>
__device__ __forceinline__ void p3_compute_aff(const uint8_t* ab, const uint8_t* sbuf, int sbs, const float* sxs,
                                               const P3Chunk<NM, NF>& ch, const uint32_t (&sbw)[NM][NF], int c, int i,
                                               int kg, int ntb, bool f16, float (&acc)[NM][NF][P3_TB][4]) {
  i32x8_t b[NM][NF];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) b[m][f] = aff_code_bytes<ak_bits(AK)>(ch.codes[m][f], kg);
#pragma unroll
  for (int tb = 0; tb < P3_TB; ++tb) {
    if (tb >= ntb) break;
    const int row = tb * 16 + i;
    const uint8_t* ar = ab + row * P3_ROWB;
    const uint4 h0 = mx::lds16(ar + ((kg ^ i) << 4));
    const uint4 h1 = mx::lds16(ar + (((4 + kg) ^ i) << 4));
    const uint4 l0 = mx::lds16(ar + (((8 + kg) ^ i) << 4));
    const uint4 l1 = mx::lds16(ar + (((12 + kg) ^ i) << 4));
    const uint32_t sa = *reinterpret_cast<const uint16_t*>(sbuf + row * sbs + (4 * c + kg) * 2);
    const i32x8_t ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
    const i32x8_t alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
    f32x4_t d[NM][NF];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f)
        d[m][f] = mfma_plane<0, true>(ahi, b[m][f], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, sa, E8M0_2P9);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) d[m][f] = mfma_plane<1, true>(alo, b[m][f], d[m][f], sa, E8M0_2P9);
    const float4 sx = *reinterpret_cast<const float4*>(sxs + c * P3_MT + tb * 16 + 4 * kg);
    const float sxv[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const float sc = scale_bits_to_f32((uint16_t)(sbw[m][f] & 0xFFFFu), f16);
        const float bi = scale_bits_to_f32((uint16_t)(sbw[m][f] >> 16), f16);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[m][f][tb][r] = fmaf(sc, d[m][f][r], fmaf(bi, sxv[r], acc[m][f][tb][r]));
      }
  }
}

// grid = slices * tiles rounded up to 8; dynamic LDS = P3_STAGES * P3_ABYTES + P3_MT * (sb + 16)
// (+ the tile's chunk sums, P3_MT * kch floats, for 2-bit banks).
template <int AK, int NM, int NF>
__global__ void __launch_bounds__(P3_THREADS) p3_kernel(MxArgs g, int slices) {
  constexpr bool Q2 = ak_fold(AK);   // affine: the group formula per group
  constexpr int GPC = ak_gpc(AK);
  extern __shared__ __align__(16) uint8_t p3_lds[];
  uint8_t* abuf = p3_lds;
  uint8_t* sbuf = p3_lds + P3_STAGES * P3_ABYTES;
  const int sbs = g.sb + 16;   // LDS row stride of the A scales (bank spread)
  float* sxs = reinterpret_cast<float*>(sbuf + P3_MT * sbs);   // affine: the tile's group sums [kch * GPC][MT]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, kg = lane >> 4;
  const int b8 = blockIdx.x >> 3;                         // sequence number on this XCD
  const int slice = b8 % slices;
  const int tile_id = (b8 / slices) * 8 + (int)(blockIdx.x & 7);
  if (tile_id >= g.tiles_n[0]) return;
  const int2 tl = g.tiles[tile_id];
  const int e = tl.x, row0 = tl.y;
  const int rows = min(P3_MT, g.offsets[e + 1] - row0);
  const int ntb = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
  const int slot = g.slot_table[e];
  constexpr int WN = 16 * NF;                            // weight rows per wave and matrix
  const int nw0 = slice * (P3_WAVES * WN) + WN * wave;   // the wave's first weight row
  // FP4: fp32 tiles in AGPRs fed by the instruction; 2-bit: fp32 in VGPRs, folded per chunk
  using AccT = typename std::conditional<Q2, float[4], f32x4_t>::type;
  AccT acc[NM][NF][P3_TB];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int tb = 0; tb < P3_TB; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[m][f][tb][r] = 0.0f;
  if (slot >= 0) {
    // affine rows hold whole groups (the bank pads the last one)
    const int groups = (g.K + ak_group(AK) - 1) / ak_group(AK);
    const int row_bytes = !Q2 ? g.K / 2 : groups * ak_group(AK) * ak_bits(AK) / 8, blocks = g.K / 32;
    // the tile's A scales into LDS for the whole K loop (rows past the tile: its last row)
    const int sq = g.sb / 16;
    for (int it = threadIdx.x; it < P3_MT * sq; it += P3_THREADS) {
      const int r = it / sq, q = it - r * sq;
      const int rr = row0 + min(r, rows - 1);
      const int src = g.a_gather ? g.a_gather[rr] : rr;
      *reinterpret_cast<uint4*>(sbuf + r * sbs + q * 16) =
          *reinterpret_cast<const uint4*>(g.as + (size_t)src * g.sb + q * 16);
    }
    if constexpr (Q2) {   // and the tile's group sums of A
      const int ns = g.kch * GPC;
      for (int it = threadIdx.x; it < P3_MT * ns; it += P3_THREADS) {
        const int ch = it / P3_MT, r = it - ch * P3_MT;
        const int rr = row0 + min(r, rows - 1);
        const int src = g.a_gather ? g.a_gather[rr] : rr;
        sxs[it] = g.asum[(size_t)src * ns + ch];
      }
    }
    // A plane sources of the lane's slots: slot S = 64 (P3_ASLOTS wave + q) + lane holds
    // row S / 16, physical 16-byte column S % 16 = logical column ^ (row % 16)
    const uint8_t* asrc[P3_ASLOTS];
#pragma unroll
    for (int q = 0; q < P3_ASLOTS; ++q) {
      const int S = 64 * (P3_ASLOTS * wave + q) + lane;
      const int r = S >> 4;
      const int col = (S & 15) ^ (r & 15);
      const int rr = row0 + min(r, rows - 1);
      const int src = g.a_gather ? g.a_gather[rr] : rr;
      asrc[q] = g.ap + (size_t)src * g.kch * P3_ROWB + col * 16;
    }
    const uint8_t* base = g.pool + (int64_t)slot * g.L.record_bytes;
    const int tq[2] = {NM == 2 ? 0 : 3, 6};   // w1, w3 (gate/up) or w2 (down)
    const uint8_t* wrow[NM][NF];
    int woff[NM], nrow[NF];   // affine: offsets in the record (< 2^31: one expert)
#pragma unroll
    for (int f = 0; f < NF; ++f) nrow[f] = min(nw0 + 16 * f + i, g.N - 1);   // rows past N: clamped (discarded)
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      woff[m] = (int)g.L.off[tq[m]];
#pragma unroll
      for (int f = 0; f < NF; ++f) wrow[m][f] = base + g.L.off[tq[m]] + (int64_t)nrow[f] * row_bytes;
    }
    // FP4 B scales: lane (i, p), p = kg = (m, f) pair, loads 32 E8M0 bytes (8 chunks) of its
    // pair's weight row i at a time, one trip ahead (NM * NF == 4); p3_scales hands them
    // out.  (16 bytes every four chunks: 3.47 against 3.39 ms per config-3 layer.)  A group
    // past the row's last block reads into what follows the tensor in the record (the
    // host checks that something does); those bytes are never used.
    static_assert(NM * NF == 4, "one (m, f) pair per lane group");
    const int pm = kg / NF, pf = kg - pm * NF;
    const uint8_t* sgp = base + g.L.off[tq[pm] + 1] + (int64_t)min(nw0 + 16 * pf + i, g.N - 1) * blocks;
    const int ngrp = (blocks + 15) / 16;
    const int nch = g.kch;
    // Affine scales and biases: lane (i, p) holds eight groups (chunks 8q .. 8q + 7) of
    // its pair's row, the scale row in sgs and the bias row in sgb (one 16-byte load
    // each, issued with chunk 8q's loads); each chunk's scale | bias << 16 goes to the
    // lanes by one shuffle per pair.  Loads per chunk and row kept the scale and bias
    // lines in L2 through the whole K loop.  A last group of eight past the row reads
    // what follows the tensor in the record (the host checks that something does).
    const int arow = min(nw0 + 16 * pf + i, g.N - 1);
    const uint8_t* sgs_p = base + g.L.off[tq[pm] + 1] + (int64_t)arow * groups * 2;
    const uint8_t* sgb_p = base + g.L.off[tq[pm] + 2] + (int64_t)arow * groups * 2;
    const int nq = (groups + 7) / 8;
    uint4 sgs, sgb;
    if constexpr (Q2) {
      sgs = *reinterpret_cast<const uint4*>(sgs_p);
      sgb = *reinterpret_cast<const uint4*>(sgb_p);
    }
    P3Chunk<NM, NF> ring[P3_STAGES];
    uint4 sgc[2], sgn[2];   // FP4 B scales of this trip's eight chunks and of the next trip's
    // every issue is unconditional (a chunk past the end re-reads the last one into a
    // stage nothing reads again), so each wait is for exactly the loads it needs
    if constexpr (!Q2) {
      sgc[0] = *reinterpret_cast<const uint4*>(sgp);
      sgc[1] = *reinterpret_cast<const uint4*>(sgp + 16 * min(1, ngrp - 1));
    }
    if constexpr (ak_bytes(AK))
      p3_issue_aff<AK, NM, NF>(abuf, asrc, base, woff, nrow, 0, kg, wave, row_bytes, ring[0]);
    else if constexpr (Q2)
      p3_issue_q2<NM, NF>(abuf, asrc, base, woff, nrow, 0, kg, wave, row_bytes, ring[0]);
    else p3_issue<NM, NF>(abuf, asrc, wrow, 0, kg, wave, row_bytes, ring[0]);
    // eight chunks per trip: A stage and code ring index u % 2, scale group buffer (u / 4) % 2
    for (int c0 = 0; c0 < nch; c0 += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u;
        // this wave's loads of chunk c have landed (its last code load is consumed
        // here; its earlier direct-to-LDS loads complete first), then every wave's
        // (affine: the first barrier also publishes the group sums stored above)
        if constexpr (Q2 && ak_bits(AK) == 2) asm volatile("" ::"v"(ring[u % 2].codes[NM - 1][NF - 1].y) : "memory");
        else asm volatile("" ::"v"(ring[u % 2].codes[NM - 1][NF - 1].w) : "memory");
        lds_sync();
        uint32_t sbw[NM][NF];
        if constexpr (Q2) {
          const int J = u >> 1, sh = 16 * (u & 1);
          const uint32_t ws = J == 0 ? sgs.x : J == 1 ? sgs.y : J == 2 ? sgs.z : sgs.w;
          const uint32_t wb = J == 0 ? sgb.x : J == 1 ? sgb.y : J == 2 ? sgb.z : sgb.w;
          const uint32_t mine = ((ws >> sh) & 0xFFFFu) | (((wb >> sh) & 0xFFFFu) << 16);
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int f = 0; f < NF; ++f)
              sbw[m][f] = (uint32_t)__shfl((int)mine, 16 * (m * NF + f) + i, 64);
          if (u == 7) {   // the next eight groups, into the registers just read
            const int q = min(c / 8 + 1, nq - 1);
            sgs = *reinterpret_cast<const uint4*>(sgs_p + 16 * q);
            sgb = *reinterpret_cast<const uint4*>(sgb_p + 16 * q);
          }
        }
        if constexpr (!Q2)
          if (u == 7) {   // the next trip's eight chunks
            sgn[0] = *reinterpret_cast<const uint4*>(sgp + 16 * min((c + 1) / 4, ngrp - 1));
            sgn[1] = *reinterpret_cast<const uint4*>(sgp + 16 * min((c + 1) / 4 + 1, ngrp - 1));
          }
        if constexpr (ak_bytes(AK))
          p3_issue_aff<AK, NM, NF>(abuf + ((u + 1) % 2) * P3_ABYTES, asrc, base, woff, nrow, min(c + 1, nch - 1), kg,
                                   wave, row_bytes, ring[(u + 1) % 2]);
        else if constexpr (Q2)
          p3_issue_q2<NM, NF>(abuf + ((u + 1) % 2) * P3_ABYTES, asrc, base, woff, nrow, min(c + 1, nch - 1), kg, wave,
                              row_bytes, ring[(u + 1) % 2]);
        else
          p3_issue<NM, NF>(abuf + ((u + 1) % 2) * P3_ABYTES, asrc, wrow, min(c + 1, nch - 1), kg, wave, row_bytes,
                           ring[(u + 1) % 2]);
        if (c < nch) {
          if constexpr (ak_bytes(AK)) {
            p3_compute_aff<AK, NM, NF>(abuf + (u % 2) * P3_ABYTES, sbuf, sbs, sxs, ring[u % 2], sbw, c, i, kg, ntb,
                                       g.L.f16, acc);
          } else if constexpr (Q2) {
            p3_compute_q2<NM, NF>(abuf + (u % 2) * P3_ABYTES, sbuf, sbs, sxs, ring[u % 2], sbw, c, i, kg, ntb,
                                  g.L.f16, acc);
          } else {
            uint32_t bs[NM][NF];
            p3_scales<NM, NF>(sgc[u / 4], u % 4, c, i, kg, blocks, bs);
            p3_compute<NM, NF>(abuf + (u % 2) * P3_ABYTES, sbuf, sbs, ring[u % 2], bs, c, i, kg, ntb, acc);
          }
        }
        if constexpr (!Q2)
          if (u == 7) {
            sgc[0] = sgn[0];
            sgc[1] = sgn[1];
          }
      }
    }
    // the re-reads issued past the end (direct-to-LDS among them) land before the
    // workgroup's LDS is released
    tile::wait_vmem();
  }
  // epilogue: lane holds rows tb*16 + 4kg + r (tile rows) x weight rows nw0 + 16f + i
  if constexpr (NM == 2) {
    // 2-bit: every wave is past its last A reads before the ring holds the h sums
    float* red = reinterpret_cast<float*>(abuf);   // [P3_WAVES][P3_MT]
    if constexpr (Q2) lds_sync();
    // h = bf16(silu(min(g, L)) * clip(u) * w), written as the planes of its 32-element
    // block (the wave's 32 weight rows are one block of h's columns)
#pragma unroll
    for (int tb = 0; tb < P3_TB; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tr = tb * 16 + 4 * kg + r;   // the same in the 16 lanes of a row group
        if (tr >= rows) continue;
        const int prow = row0 + tr;
        const float wr = g.row_w[prow];
        float hv[NF];
        float m = 0.0f;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          float gv = round_bf16(acc[0][f][tb][r]);
          float uv = round_bf16(acc[1][f][tb][r]);
          if (g.limit > 0.0f) {
            uv = fminf(fmaxf(uv, -g.limit), g.limit);
            gv = fminf(gv, g.limit);
          }
          hv[f] = nw0 + 16 * f + i < g.N ? round_bf16((silu_f32(gv) * uv) * wr) : 0.0f;
          m = fmaxf(m, fabsf(hv[f]));
        }
        m = mx::row16_max(m);
        const int E = plane_exp(m);
        const float inv = __uint_as_float((uint32_t)(127 - E) << 23);
        uint8_t* dst = g.hp + (size_t)prow * g.hkch * P3_ROWB;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const float s = hv[f] * inv;
          const uint32_t hi = mx::f32_to_e4m3(s);
          const uint32_t lo = mx::f32_to_e4m3((s - mx::e4m3_to_f32(hi)) * 16.0f);
          const int n = nw0 + 16 * f + i;
          uint8_t* p = dst + (n >> 7) * P3_ROWB + (n & 127);
          p[0] = (uint8_t)hi;
          p[128] = (uint8_t)lo;
        }
        if (i == 0) {
          const uint32_t sc = (uint32_t)(E + 127) | ((uint32_t)(E + 123) << 8);
          *reinterpret_cast<uint16_t*>(g.hs + (size_t)prow * g.hsb + (nw0 / 32) * 2) = (uint16_t)sc;
        }
        if constexpr (Q2) {   // the wave's 32 h values of the row, summed (f, then the 16 lanes)
          float hsv = 0.0f;
#pragma unroll
          for (int f = 0; f < NF; ++f) hsv = hsv + hv[f];
          hsv = row16_sum(hsv);
          if (i == 0) red[wave * P3_MT + tr] = hsv;
        }
      }
    if constexpr (Q2) {   // the workgroup's 128 columns are one chunk of h: its group sums per row,
                          // waves in order (G = 64: waves 0, 1 and 2, 3)
      lds_sync();
      if ((int)threadIdx.x < rows) {
        const int tr = threadIdx.x;
#pragma unroll
        for (int h = 0; h < GPC; ++h) {
          float t = 0.0f;
#pragma unroll
          for (int w = h * P3_WAVES / GPC; w < (h + 1) * P3_WAVES / GPC; ++w) t = t + red[w * P3_MT + tr];
          g.hsum[(size_t)(row0 + tr) * g.hkch * GPC + slice * GPC + h] = t;
        }
      }
    }
  } else {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int n = nw0 + 16 * f + i;
      if (n >= g.N) continue;
#pragma unroll
      for (int tb = 0; tb < P3_TB; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tr = tb * 16 + 4 * kg + r;
          if (tr >= rows) continue;
          const int rr = row0 + tr;
          g.y[((size_t)g.row_token[rr] * g.k + g.row_slot[rr]) * g.N + n] = f32_to_bf16(acc[0][f][tb][r]);
        }
    }
  }
}

}  // namespace

// Workspace of the block-scaled prefill beyond the tile list: x planes [T][D/128][256]
// and scales [T][sb(D)], h planes [rows][F_pad/128][256] and scales [rows][sb(F_pad)],
// affine group sums of x [T][D/64 or D/128] and of h [rows][2 or 1 per 128 columns].
size_t prefill_mx_ws_bytes(int T, int k, int D, int F) {
  const size_t rows = (size_t)T * k;
  const int fch = (F + 127) / 128;
  auto a256 = [](size_t v) { return (v + 255) & ~size_t(255); };
  return a256((size_t)T * D * 2) + a256((size_t)T * scale_row_bytes(D)) + a256(rows * fch * P3_ROWB) +
         a256(rows * scale_row_bytes(fch * 128)) + a256((size_t)T * (D / 64) * 4) + a256(rows * fch * 2 * 4);
}

// Shapes and slot layouts the kernels take.  Their B-scale loads read 16 bytes per
// row at a time; when a scale row is not a whole number of 16-byte groups, the last
// group of the tensor's last row reads up to 15 bytes past the tensor, which must
// still lie inside the slot record.
// Rows per tile of the tile list these kernels take.
int prefill_mx_mt() { return P3_MT; }

bool prefill_mx_supported(int D, int F, const decode::Layout& L) {
  if (!(D % 128 == 0 && D >= 512 && D <= 8192 && F % 32 == 0 && F >= 512 && F <= 8192)) return false;
  auto room = [&](int t, int64_t rows, int blocks) {
    return blocks % 16 == 0 || L.off[t] + rows * blocks + 16 <= L.record_bytes;
  };
  return room(1, F, D / 32) && room(7, F, D / 32) && room(4, D, F / 32);
}

// Affine scales and biases are read eight groups at a time: where a row's group count
// is not a multiple of eight, the last load of the tensor's last row reads up to 16
// bytes past the tensor, which must still lie inside the slot record.
static bool affine_scale_room(int group, int D, int F, const decode::Layout& L) {
  auto room = [&](int t, int64_t rows, int groups) {
    return groups % 8 == 0 || L.off[t] + rows * groups * 2 + 16 <= L.record_bytes;
  };
  const int gd = (D + group - 1) / group, gf = (F + group - 1) / group;
  return room(1, F, gd) && room(2, F, gd) && room(7, F, gd) && room(8, F, gd) && room(4, D, gf) && room(5, D, gf);
}

// 2-bit g128 banks: any shape of the FP4 envelope (the rows' groups are padded to whole
// chunks in the bank).
bool prefill_mx_q2_supported(int D, int F, const decode::Layout& L) {
  return D % 128 == 0 && D >= 512 && D <= 8192 && F % 32 == 0 && F >= 512 && F <= 8192 &&
         affine_scale_room(128, D, F, L);
}

namespace {

template <int AK>
int launch_p3(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L, const int32_t* slot_table,
              const int32_t* offsets, const int2* tiles, const int32_t* tiles_n, int max_tiles,
              const int32_t* row_token, const int32_t* row_slot, const float* row_w, int D, int F, int k, float limit,
              uint8_t* ws, uint16_t* y, hipStream_t s) {
  auto a256 = [](size_t v) { return (v + 255) & ~size_t(255); };
  const size_t rows = (size_t)T * k;
  const int fch = (F + 127) / 128;
  const int sbx = scale_row_bytes(D), sbh = scale_row_bytes(fch * 128);
  uint8_t* xp = ws;
  uint8_t* xs = xp + a256((size_t)T * D * 2);
  uint8_t* hp = xs + a256((size_t)T * sbx);
  uint8_t* hs = hp + a256(rows * fch * P3_ROWB);
  float* xsum = reinterpret_cast<float*>(hs + a256(rows * sbh));
  float* hsum = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(xsum) + a256((size_t)T * (D / 64) * 4));
  constexpr bool Q2 = ak_fold(AK);
  constexpr int GPC = ak_gpc(AK);
  const int64_t groups = (int64_t)T * D / 8;
  hipLaunchKernelGGL(x_planes_rows_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, x, T, D, xp, xs,
                     sbx, Q2 ? xsum : nullptr, 128 / GPC);
  int rc = check_launch("x_planes_rows_kernel");
  if (rc) return rc;
  const int tiles8 = (max_tiles + 7) / 8 * 8;
  MxArgs gu{xp, xs, sbx, D / 128, row_token, pool, L, slot_table, offsets, tiles, tiles_n, row_token, row_slot,
            row_w, D, F, k, limit, hp, hs, sbh, fch, nullptr, xsum, hsum};
  const int s_gu = (fch * 128) / (P3_WAVES * 32);   // h's padded columns, 128 per workgroup
  const size_t lds_gu = (size_t)P3_STAGES * P3_ABYTES + (size_t)P3_MT * (sbx + 16) +
                        (Q2 ? (size_t)P3_MT * (D / 128) * GPC * 4 : 0);
  MxArgs dn{hp, hs, sbh, fch, nullptr, pool, L, slot_table, offsets, tiles, tiles_n, row_token, row_slot, row_w,
            F, D, k, limit, nullptr, nullptr, 0, 0, y, hsum, nullptr};
  const int s_dn = (D + P3_WAVES * 64 - 1) / (P3_WAVES * 64);
  const size_t lds_dn = (size_t)P3_STAGES * P3_ABYTES + (size_t)P3_MT * (sbh + 16) +
                        (Q2 ? (size_t)P3_MT * fch * GPC * 4 : 0);
  // affine fp8 codes in groups of 64: the 32 x 32 x 64 kernels (prefill_affine_mx.hip)
  if constexpr (ak_bytes(AK) && ak_group(AK) == 64) {
    return launch_prefill_affine_g64(AK, gu, s_gu, lds_gu, dn, s_dn, lds_dn, tiles8, s);
  } else {
  auto kgu = p3_kernel<AK, 2, 2>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kgu), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_gu) != hipSuccess)
    return fail(CACHALOT_EHIP, "prefill (block-scaled): cannot grant %zu bytes of LDS", lds_gu);
  hipLaunchKernelGGL(kgu, dim3(s_gu * tiles8), dim3(P3_THREADS), lds_gu, s, gu, s_gu);
  rc = check_launch("p3_kernel<2,2>");
  if (rc) return rc;
  auto kdn = p3_kernel<AK, 1, 4>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kdn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_dn) != hipSuccess)
    return fail(CACHALOT_EHIP, "prefill (block-scaled): cannot grant %zu bytes of LDS", lds_dn);
  hipLaunchKernelGGL(kdn, dim3(s_dn * tiles8), dim3(P3_THREADS), lds_dn, s, dn, s_dn);
  return check_launch("p3_kernel<1,4>");
  }
}

}  // namespace

// tiles / tiles_n: the 64-row tile list (tile_list_kernel with MT = 64), max_tiles its bound.
int launch_prefill_mx(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L,
                      const int32_t* slot_table, const int32_t* offsets, const int2* tiles, const int32_t* tiles_n,
                      int max_tiles, const int32_t* row_token, const int32_t* row_slot, const float* row_w, int D,
                      int F, int k, float limit, uint8_t* ws, uint16_t* y, hipStream_t s) {
  return launch_p3<AK_FP4>(x, T, pool, L, slot_table, offsets, tiles, tiles_n, max_tiles, row_token, row_slot, row_w,
                          D, F, k, limit, ws, y, s);
}

// The same launches over a 2-bit g128 bank.
int launch_prefill_mx_q2(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L,
                         const int32_t* slot_table, const int32_t* offsets, const int2* tiles,
                         const int32_t* tiles_n, int max_tiles, const int32_t* row_token, const int32_t* row_slot,
                         const float* row_w, int D, int F, int k, float limit, uint8_t* ws, uint16_t* y,
                         hipStream_t s) {
  return launch_p3<AK_Q2>(x, T, pool, L, slot_table, offsets, tiles, tiles_n, max_tiles, row_token, row_slot, row_w,
                          D, F, k, limit, ws, y, s);
}

// The other affine widths the kernels take: 2-bit codes in groups of 64, 3- and 4-bit
// codes in groups of 64 or 128 (groups of 32 would need four instructions per plane
// and chunk), in the shapes of the FP4 envelope with F a multiple of 64.
bool prefill_mx_aff_supported(int bits, int group, int D, int F, const decode::Layout& L) {
  const bool kind = (bits == 2 && group == 64) || ((bits == 3 || bits == 4) && (group == 64 || group == 128));
  return kind && D % 128 == 0 && D >= 512 && D <= 8192 && F % 64 == 0 && F >= 512 && F <= 8192 &&
         affine_scale_room(group, D, F, L);
}

int launch_prefill_mx_aff(int bits, int group, const uint16_t* x, int T, const uint8_t* pool,
                          const decode::Layout& L, const int32_t* slot_table, const int32_t* offsets,
                          const int2* tiles, const int32_t* tiles_n, int max_tiles, const int32_t* row_token,
                          const int32_t* row_slot, const float* row_w, int D, int F, int k, float limit, uint8_t* ws,
                          uint16_t* y, hipStream_t s) {
#define CACHALOT_P3AFF(B, G)                                                                                       \
  if (bits == B && group == G)                                                                                     \
    return launch_p3<ak_aff(B, G)>(x, T, pool, L, slot_table, offsets, tiles, tiles_n, max_tiles, row_token,      \
                                   row_slot, row_w, D, F, k, limit, ws, y, s);
  CACHALOT_P3AFF(2, 64) CACHALOT_P3AFF(3, 64) CACHALOT_P3AFF(3, 128) CACHALOT_P3AFF(4, 64) CACHALOT_P3AFF(4, 128)
#undef CACHALOT_P3AFF
  return fail(CACHALOT_EINVAL, "prefill (block-scaled): %d-bit codes in groups of %d", bits, group);
}

}  // namespace cachalot
