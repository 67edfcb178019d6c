// Decode (one token) over affine banks of the other widths -- 3- and 4-bit codes in
// groups of 32, 64 or 128, 2-bit codes in groups of 32 or 64, bf16 or fp16 scales
// (the oQ3e bank is 3-bit g64 fp16, src/cachalot/model/expert_affine.py:1-10) -- on
// the block-scaled fp8 x fp4 matrix cores, in the two launches of the 2-bit g128
// decode (decode_q2_mx.hip) and with the same arithmetic: the group formula
// s * sum(x q) + b * sum(x) per group (minimax/codes_qmv.py:86-100), bf16 g, u, h
// and y_e, experts summed in route order from zero (expert_affine.py:65-81,117-152).
//
// The group-separated layout of mx_tile.h, generalised: an item is (16-row tile,
// quad of four groups), lane group kg of the B operand carrying group 4 q + kg of
// its weight row, 32 codes per instruction, G / 32 instructions per group.  A row
// r = 4 kg' + 2 h + p of the A operand carries plane p of piece h of the same 32
// codes of group 4 q + kg'; x and h stay in the 128-element plane blocks the
// router and the gate/up epilogue write, a group of G < 128 codes being chunks
// cb .. cb + G/32 - 1 of its block (the scale lanes shift their four chunk scales
// so that the instruction's byte select picks chunk cb + step).
//
// Codes as fp4 operands (E2M1 of q / 2 with scale 2, as the 2-bit path):
//   2-bit: the 2-bit spread (mx_tile.h q2_spread), one instruction per step;
//   3- and 4-bit: q = 4 (q >> 2) + (q & 3), two instructions per step sharing the
//     A operand -- the low two bits with B scale 2, the high bits (0..3) with B
//     scale 8.  The codes of a step are first put one per nibble in natural order
//     (3-bit: each 24-bit run of eight codes spread to nibbles), then into the
//     plane blocks' element order (0, 2, .., 14, 1, 3, .., 15 per 16 codes) by a
//     byte permute.  Every product is exact; each dot product of the instruction
//     holds one 16-value plane piece (values within 2^13 of each other) times
//     codes of at most 12, so the instruction's internal sum stays exact as in the
//     2-bit path.
#include "decode_common.h"
#include "mfma_tile.h"
#include "mx_tile.h"

namespace cachalot {

int launch_x_planes(const uint16_t* x, int D, uint8_t* xplanes, hipStream_t s);   // decode_q2_mx.hip

namespace {

using namespace decode;
using mx::a_role;
using mx::ARole;
using mx::dot4;
using mx::f32x4_t;
using mx::i32x8_t;
using mx::PB_BYTES;
using mx::PB_SCALE;
using mx::PB_SUM;
using tile::copy_to_lds_untracked;
using tile::waitcnt_vm;

constexpr int AG_THREADS = 256;
constexpr int AG_WAVES = AG_THREADS / 64;
constexpr int AD_THREADS = 768;
constexpr int AD_WAVES = AD_THREADS / 64;
constexpr int AM_MAX_D = 5120;                 // gate/up K
constexpr int AM_MAX_F = 3072;                 // down K
constexpr int AM_MAX_GT = AM_MAX_D / 128;      // x plane blocks
constexpr int AM_MAX_GKB = AM_MAX_F / 128;     // h plane blocks per expert
constexpr uint32_t E8M0_TWO = 128u;            // 2^1
constexpr uint32_t E8M0_EIGHT = 130u;          // 2^3

template <int BITS, int G>
struct Geo {
  static constexpr int STEPS = G / 32;                  // instructions (per part) per group
  static constexpr int W = G * BITS / 32;               // u32 words of one group of one row
  static constexpr int LDI = W % 4 == 0 ? W / 4 : (W % 2 == 0 ? W / 2 : W);   // load instructions per group
};

// The W words of one group of one row (16-, 8- or 4-byte loads as the group's
// alignment allows: a group starts at a multiple of W * 4 bytes of a 16-byte aligned row).
template <int W>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t (&w)[W]) {
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else if constexpr (W % 2 == 0) {
#pragma unroll
    for (int i = 0; i < W / 2; ++i) {
      const uint2 v = reinterpret_cast<const uint2*>(p)[i];
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = reinterpret_cast<const uint32_t*>(p)[i];
  }
}

// 3- and 4-bit codes go to the matrix cores in natural order (nibble j of B word t =
// code 8 t + j of the lane's 32), so the kernels put their LDS copy of the plane blocks
// in natural order too: a piece's 16 bytes hold its even elements, then its odd ones
// (the order the 2-bit spread yields), and each wave re-orders the 16-byte runs it
// copied itself once they have landed.  Run r of `bytes` copied by copy_to_lds_untracked
// with (part, parts); only the data runs (the first 256 bytes of a block) move.
__device__ __forceinline__ void planes_natural_own(uint8_t* planes, int bytes, int part, int parts, int lane) {
  asm volatile("" ::: "memory");   // after the caller's wait for the copies
  for (int c = part * 1024 + 16 * lane; c < bytes; c += parts * 1024) {
    if (c % PB_BYTES >= PB_SCALE) continue;
    uint4* p = reinterpret_cast<uint4*>(planes + c);
    const uint4 v = *p;   // bytes 0..7: elements 0, 2, .., 14; bytes 8..15: 1, 3, .., 15
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05010400u);   // elements 0, 1, 2, 3
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07030602u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05010400u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07030602u);
    *p = o;
  }
}

// B operands of step s of a group whose words are w: `lo` (and for 3 / 4 bits `hi`).
// 2-bit codes in the planes' piece order, 3- and 4-bit codes in natural order.
template <int BITS, int W>
__device__ __forceinline__ void step_operands(const uint32_t (&w)[W], int s, i32x8_t& lo, i32x8_t& hi) {
  if constexpr (BITS == 2) {
    lo = mx::q2_spread(w[2 * s], w[2 * s + 1]);
  } else {
    uint32_t n[4];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int t = 0; t < 4; ++t) n[t] = w[4 * s + t];
    } else {
      const uint32_t w0 = w[3 * s], w1 = w[3 * s + 1], w2 = w[3 * s + 2];
      n[0] = mx::spread3(w0 & 0xFFFFFFu);
      n[1] = mx::spread3(__builtin_amdgcn_alignbit(w1, w0, 24) & 0xFFFFFFu);
      n[2] = mx::spread3(__builtin_amdgcn_alignbit(w2, w1, 16) & 0xFFFFFFu);
      n[3] = mx::spread3(w2 >> 8);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo[t] = (int)(n[t] & 0x33333333u);
      hi[t] = (int)((n[t] >> 2) & 0x33333333u);
      lo[t + 4] = 0;
      hi[t + 4] = 0;
    }
  }
}

// Where group g's elements sit in the plane blocks: block g G / 128, first chunk
// (32 elements) cb = (g G / 32) mod 4.
template <int G>
__device__ __forceinline__ int group_block(int g) { return (g * G) >> 7; }
template <int G>
__device__ __forceinline__ int group_chunk(int g) { return ((g * G) >> 5) & 3; }

// Sum of a group's piece sums (pieces 2 cb .. 2 cb + 2 G / 32 - 1, in order).
template <int G>
__device__ __forceinline__ float group_xsum(const uint8_t* blk, int cb) {
  const float4 a = *reinterpret_cast<const float4*>(blk + PB_SUM);
  const float4 b = *reinterpret_cast<const float4*>(blk + PB_SUM + 16);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float s = 0.0f;
#pragma unroll
  for (int p = 0; p < 2 * (G / 32); ++p) s = s + v[min(2 * cb + p, 7)];
  return s;
}

// One item: the lane's codes of the item's group for one or two matrices, the A
// operand stepped through the group's chunks.  Returns the accumulators.
template <int BITS, int G, int NMAT>
__device__ __forceinline__ void item_mfma(const uint8_t* ablk, int acb, const ARole& ro,
                                          const uint32_t (&c0)[Geo<BITS, G>::W],
                                          const uint32_t (&c1)[Geo<BITS, G>::W], f32x4_t& acc0, f32x4_t& acc1) {
  using Gm = Geo<BITS, G>;
  i32x8_t av = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t sav = 0x7F7F7F7Fu;
  mx::chain_scales(sav, ablk, ro);
  if (ro.scale) sav >>= 8 * acb;
  acc0 = mx::zero_acc();
  acc1 = mx::zero_acc();
#pragma unroll
  for (int s = 0; s < Gm::STEPS; ++s) {
    mx::chain_load_step(av, ablk, ro, acb + s);
    i32x8_t lo0, hi0, lo1, hi1;
    step_operands<BITS>(c0, s, lo0, hi0);
    acc0 = mx::mfma_fp8_fp4_sel(s, av, lo0, acc0, sav, E8M0_TWO);
    if constexpr (NMAT == 2) {
      step_operands<BITS>(c1, s, lo1, hi1);
      acc1 = mx::mfma_fp8_fp4_sel(s, av, lo1, acc1, sav, E8M0_TWO);
    }
    if constexpr (BITS != 2) {
      acc0 = mx::mfma_fp8_fp4_sel(s, av, hi0, acc0, sav, E8M0_EIGHT);
      if constexpr (NMAT == 2) acc1 = mx::mfma_fp8_fp4_sel(s, av, hi1, acc1, sav, E8M0_EIGHT);
    }
  }
}

template <int G>
struct AGuLds {
  uint8_t planes[AM_MAX_GT * PB_BYTES];
  uint16_t sc[4][16 * (AM_MAX_D / G)];   // s1, b1, s3, b3 of the tile's 16 rows (one contiguous run each)
  float red[AM_MAX_D / G / 4][2][16];
  int top_i[KMAX], top_s[KMAX];
  float top_v[KMAX], top_w[KMAX];
  int slot;
  float wexp;
};

// grid.x = k * F / 16: one workgroup = one expert x one 16-row tile of W1 and W3.
// MAXM = items per wave (ceil(D / G / 16)); every item's codes are loaded up front.
template <int BITS, int G, int MAXM>
__global__ void __launch_bounds__(AG_THREADS) amx_gate_up_kernel(const uint8_t* __restrict__ xplanes,
                                                                 const uint8_t* __restrict__ pool, Layout L,
                                                                 ExpertSource src, int D, int F, float limit,
                                                                 uint8_t* __restrict__ hid,
                                                                 int32_t* __restrict__ ws_slots,
                                                                 float* __restrict__ ws_w) {
  using Gm = Geo<BITS, G>;
  __shared__ __align__(16) AGuLds<G> s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int GT = D / 128, GN = D / G, NQ = GN / 4;
  const int GK = (F + 127) / 128, FT = F / 16;
  const int bid = blockIdx.x;
  const int e = bid / FT;
  const int tile = bid - e * FT;
  const int row0 = tile * 16;
  const int rw = bid & (AG_WAVES - 1);   // the routing wave

  // ---- 0. routing wave: the expert's slot; the others: x's plane blocks into LDS
  if (wave == rw) {
    const int slot = route_slot(src, ws_slots, e, s.top_i, s.top_v, s.top_s);
    if (lane == 0) s.slot = slot;
    tile::wait_vmem();
  } else {
    copy_to_lds_untracked(xplanes, s.planes, GT * PB_BYTES, wave < rw ? wave : wave - 1, AG_WAVES - 1, lane);
    tile::wait_vmem();
    if constexpr (BITS != 2) planes_natural_own(s.planes, GT * PB_BYTES, wave < rw ? wave : wave - 1, AG_WAVES - 1, lane);
  }
  lds_sync();
  const int slot = __builtin_amdgcn_readfirstlane(s.slot);
  const bool live = slot >= 0;
  const ARole ro = a_role(lane);

  // ---- 1. loads: wave w copies the tile's run of scale / bias tensor w, then its
  //         items' codes (unconditional, clamped: a missing expert reads slot 0's)
  uint32_t c1[MAXM][Gm::W], c3[MAXM][Gm::W];
  {
    const uint8_t* base = pool + (int64_t)max(slot, 0) * L.record_bytes;
    const int64_t toff = wave == 0 ? L.off[1] : wave == 1 ? L.off[2] : wave == 2 ? L.off[7] : L.off[8];
    copy_to_lds_untracked(base + toff + (int64_t)row0 * GN * 2, reinterpret_cast<uint8_t*>(s.sc[wave]), 32 * GN, 0,
                          1, lane);
    const int rowb = GN * Gm::W * 4;
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int q = min(wave + AG_WAVES * m, NQ - 1);
      const int off = (row0 + j) * rowb + (4 * q + kg) * (Gm::W * 4);
      load_words<Gm::W>(base + L.off[0] + off, c1[m]);
      load_words<Gm::W>(base + L.off[6] + off, c3[m]);
    }
  }
  if (src.scores != nullptr && wave == rw) {
    const float w = route_weight(src, ws_w, e, s.top_v, s.top_w);
    if (lane == 0) s.wexp = w;
  }
  // the run copy, issued before the code loads, has landed; the codes stay in flight
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * MAXM * Gm::LDI));
  lds_sync();

  // ---- 2. items
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    const int q = wave + AG_WAVES * m;
    if (!live || q >= NQ) break;
    const int ga = 4 * q + ro.kgR;   // the group whose x this lane's A data carries
    f32x4_t a1, a3;
    item_mfma<BITS, G, 2>(s.planes + group_block<G>(ga) * PB_BYTES, group_chunk<G>(ga), ro, c1[m], c3[m], a1, a3);
    const int gl = 4 * q + kg;       // the lane's own group
    const float sx = group_xsum<G>(s.planes + group_block<G>(gl) * PB_BYTES, group_chunk<G>(gl));
    const int si = j * GN + gl;
    const float v1 = scale_bits_to_f32(s.sc[0][si], L.f16) * dot4(a1) + scale_bits_to_f32(s.sc[1][si], L.f16) * sx;
    const float v3 = scale_bits_to_f32(s.sc[2][si], L.f16) * dot4(a3) + scale_bits_to_f32(s.sc[3][si], L.f16) * sx;
    const float r1 = tile::sum_lane_groups(v1);
    const float r3 = tile::sum_lane_groups(v3);
    if (lane < 16) {
      s.red[q][0][lane] = r1;
      s.red[q][1][lane] = r3;
    }
  }
  lds_sync();

  // ---- 3. epilogue (16 lanes of wave 0): h for the tile's rows as one plane piece
  if (tid < 16) {
    if (tid == 0 && (src.idx || src.scores) && tile == 0) ws_slots[e] = slot;
    const float wexp = src.scores != nullptr ? s.wexp : expert_weight(src, ws_w, e);
    if (src.scores != nullptr) {
      if (tile == 0 && tid == 0) ws_w[e] = wexp;
      if (bid == 0 && tid < src.k) {
        if (src.idx_out) src.idx_out[tid] = s.top_i[tid];
        if (src.w_out) src.w_out[tid] = s.top_w[tid];
      }
    }
    float hv = 0.0f;
    if (live) {
      float g = 0.0f, u = 0.0f;
      for (int q = 0; q < NQ; ++q) {
        g = g + s.red[q][0][tid];
        u = u + s.red[q][1][tid];
      }
      g = round_bf16(g);
      u = round_bf16(u);
      if (limit > 0.0f) {
        u = fminf(fmaxf(u, -limit), limit);
        g = fminf(g, limit);
      }
      hv = round_bf16((silu_f32(g) * u) * wexp);
    }
    const mx::PieceCode pc = mx::encode_piece(hv);
    const int pp = tile & 7;
    uint8_t* blk = hid + ((int64_t)e * GK + (tile >> 3)) * PB_BYTES;
    blk[mx::pb_data(pp, 0) + mx::piece_pos(tid)] = (uint8_t)pc.hi;
    blk[mx::pb_data(pp, 1) + mx::piece_pos(tid)] = (uint8_t)pc.lo;
    if (tid == 0) {
      blk[mx::pb_scale(pp, 0)] = (uint8_t)pc.scales;
      blk[mx::pb_scale(pp, 1)] = (uint8_t)(pc.scales >> 8);
      *reinterpret_cast<float*>(blk + PB_SUM + 4 * pp) = pc.sum;
    }
    if (tile == FT - 1) {   // pieces of the last block past F: zeros (consumers read whole steps)
      for (int z = pp + 1; z < mx::PIECES; ++z) {
        blk[mx::pb_data(z, 0) + tid] = 0;
        blk[mx::pb_data(z, 1) + tid] = 0;
        if (tid == 0) {
          blk[mx::pb_scale(z, 0)] = 127;
          blk[mx::pb_scale(z, 1)] = 127;
          *reinterpret_cast<float*>(blk + PB_SUM + 4 * z) = 0.0f;
        }
      }
    }
  }
}

template <int G>
struct ADnLds {
  uint8_t planes[KMAX * AM_MAX_GKB * PB_BYTES];
  uint16_t sc[KMAX][2][16 * (AM_MAX_F / G)];   // per expert: s2, b2 runs of the tile's rows
  float red[KMAX][(AM_MAX_F / G + 3) / 4][16];
  float y[KMAX][16];
};

// grid.x = D / 16: one 768-thread workgroup = one 16-row tile of W2 for all k experts;
// items (expert, quad of four groups along F) dealt round-robin to the 12 waves.
template <int BITS, int G, int MAXM>
__global__ void __launch_bounds__(AD_THREADS) amx_down_kernel(const uint8_t* __restrict__ pool, Layout L,
                                                              const int32_t* __restrict__ ws_slots, int D, int F,
                                                              int k, const uint8_t* __restrict__ hid,
                                                              const uint16_t* __restrict__ addend,
                                                              float* __restrict__ routed, uint16_t* __restrict__ out) {
  using Gm = Geo<BITS, G>;
  __shared__ __align__(16) ADnLds<G> s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int GK = (F + G - 1) / G, GKB = (F + 127) / 128, NQ2 = (GK + 3) / 4;
  const int row0 = blockIdx.x * 16;
  const int n_items = k * NQ2;

  // ---- 0. the hidden plane blocks, the scale / bias runs, then the wave's W2 codes
  copy_to_lds_untracked(hid, s.planes, k * GKB * PB_BYTES, wave, AD_WAVES, lane);
  // the tile's addend, read now (every lane loads, no branch); without one the read
  // lands in the workspace (h planes, then x's: at least 2 D bytes) and is unused
  const uint16_t add_bits = (addend != nullptr ? addend : reinterpret_cast<const uint16_t*>(hid))[row0 + (tid & 15)];
  int eslot[KMAX];
#pragma unroll
  for (int e = 0; e < KMAX; ++e) eslot[e] = ws_slots[e];
  for (int r = wave; r < 2 * k; r += AD_WAVES) {
    int ps = eslot[0];
#pragma unroll
    for (int e = 1; e < KMAX; ++e) ps = e == (r >> 1) ? eslot[e] : ps;
    ps = max(ps, 0);   // a missing expert's rows are never used
    const uint8_t* src = pool + (int64_t)ps * L.record_bytes + ((r & 1) ? L.off[5] : L.off[4]) +
                         (int64_t)row0 * GK * 2;
    copy_to_lds_untracked(src, reinterpret_cast<uint8_t*>(s.sc[r >> 1][r & 1]), 32 * GK, 0, 1, lane);
  }
  uint32_t c2[MAXM][Gm::W];
  int it_e[MAXM], it_q[MAXM];
  bool on[MAXM];
  const int rowb = GK * Gm::W * 4;
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    const int it = wave + AD_WAVES * m;
    const int itc = min(it, n_items - 1);
    it_e[m] = itc / NQ2;
    it_q[m] = itc - it_e[m] * NQ2;
    int slot = eslot[0];
#pragma unroll
    for (int e = 1; e < KMAX; ++e) slot = e == it_e[m] ? eslot[e] : slot;
    on[m] = it < n_items && slot >= 0;
    const int g2 = min(4 * it_q[m] + kg, GK - 1);
    const uint8_t* base = pool + (int64_t)max(slot, 0) * L.record_bytes;
    load_words<Gm::W>(base + L.off[3] + (int64_t)(row0 + j) * rowb + g2 * (Gm::W * 4), c2[m]);
  }
  // the copies (issued first) have landed; the codes stay in flight
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(MAXM * Gm::LDI));
  if constexpr (BITS != 2) planes_natural_own(s.planes, k * GKB * PB_BYTES, wave, AD_WAVES, lane);
  lds_sync();

  // ---- 1. items
  const ARole ro = a_role(lane);
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    if (wave + AD_WAVES * m >= n_items) break;
    const int e = it_e[m], q2 = it_q[m];
    const int ga = min(4 * q2 + ro.kgR, GK - 1);
    f32x4_t acc, unused;
    item_mfma<BITS, G, 1>(s.planes + (e * GKB + group_block<G>(ga)) * PB_BYTES, group_chunk<G>(ga), ro, c2[m], c2[m],
                          acc, unused);
    const int gl = 4 * q2 + kg;
    const int glc = min(gl, GK - 1);
    const float sh = group_xsum<G>(s.planes + (e * GKB + group_block<G>(glc)) * PB_BYTES, group_chunk<G>(glc));
    const int si = j * GK + glc;
    float v = gl < GK ? scale_bits_to_f32(s.sc[e][0][si], L.f16) * dot4(acc) +
                            scale_bits_to_f32(s.sc[e][1][si], L.f16) * sh
                      : 0.0f;
    v = tile::sum_lane_groups(v);
    if (on[m] && lane < 16) s.red[e][q2][lane] = v;
  }
  lds_sync();

  // ---- 2. per expert: the row values rounded to bf16; then the route-order sum
  if (tid < 16 * k) {
    const int e = tid >> 4, r = tid & 15;
    float y = 0.0f;
    for (int q2 = 0; q2 < NQ2; ++q2) y = y + s.red[e][q2][r];
    int se = eslot[0];
#pragma unroll
    for (int x = 1; x < KMAX; ++x) se = x == e ? eslot[x] : se;
    s.y[e][r] = se >= 0 ? round_bf16(y) : 0.0f;
  }
  lds_sync();
  if (tid < 16) {
    const int n = row0 + tid;
    float total = 0.0f;
    for (int e = 0; e < k; ++e) total = total + s.y[e][tid];
    if (routed) routed[n] = total;
    if (out) out[n] = f32_to_bf16(addend ? total + bf16_to_f32(add_bits) : total);
  }
}

template <int BITS, int G>
int launch_pair(const uint8_t* xplanes, const uint8_t* pool, const Layout& L, const ExpertSource& src,
                int32_t* ws_slots, float* ws_w, int D, int F, int k, float limit, const uint16_t* addend,
                float* routed, uint16_t* out, uint8_t* hid, hipStream_t s) {
  const int mg = (D / G / 4 + AG_WAVES - 1) / AG_WAVES;
  constexpr int MG4 = 4096 / G / 16, MG5 = AM_MAX_D / G / 16 + (AM_MAX_D % (16 * G) ? 1 : 0);
  const dim3 grid_gu(k * (F / 16));
  if (mg <= MG4)
    hipLaunchKernelGGL((amx_gate_up_kernel<BITS, G, MG4>), grid_gu, dim3(AG_THREADS), 0, s, xplanes, pool, L, src, D,
                       F, limit, hid, ws_slots, ws_w);
  else
    hipLaunchKernelGGL((amx_gate_up_kernel<BITS, G, MG5>), grid_gu, dim3(AG_THREADS), 0, s, xplanes, pool, L, src, D,
                       F, limit, hid, ws_slots, ws_w);
  if (int rc = check_launch("amx_gate_up_kernel")) return rc;
  const int GK = (F + G - 1) / G;
  const int md = (k * ((GK + 3) / 4) + AD_WAVES - 1) / AD_WAVES;
  // k = 6 at F = 2880: 3 (g128), 6 (g64), 12 (g32) items per wave; up to k = 8 at F = 3072
  constexpr int MD6 = G == 128 ? 3 : G == 64 ? 6 : 12;
  constexpr int MD8 = (KMAX * ((AM_MAX_F / G + 3) / 4) + AD_WAVES - 1) / AD_WAVES;
  if (md <= MD6)
    hipLaunchKernelGGL((amx_down_kernel<BITS, G, MD6>), dim3(D / 16), dim3(AD_THREADS), 0, s, pool, L, ws_slots, D, F,
                       k, hid, addend, routed, out);
  else
    hipLaunchKernelGGL((amx_down_kernel<BITS, G, MD8>), dim3(D / 16), dim3(AD_THREADS), 0, s, pool, L, ws_slots, D, F,
                       k, hid, addend, routed, out);
  return check_launch("amx_down_kernel");
}

}  // namespace

// The widths and shapes these kernels take: 3- and 4-bit codes in groups of 32, 64
// or 128 and 2-bit codes in groups of 32 or 64 (2-bit g128 has decode_q2_mx.hip);
// D a multiple of 4 G and of 1024 up to 5120 (x in whole plane blocks and quads),
// F a multiple of 16 up to 3072, k <= 8.
bool affine_mx_supported(int bits, int group, int D, int F, int k) {
  const bool width = (bits == 3 || bits == 4) ? (group == 32 || group == 64 || group == 128)
                                              : (bits == 2 && (group == 32 || group == 64));
  return width && D % 1024 == 0 && D <= AM_MAX_D && F % 16 == 0 && F >= 16 && F <= AM_MAX_F && k >= 1 &&
         k <= KMAX;
}

// Workspace beyond the slots and weights: the hidden plane blocks of k experts, then x's.
size_t affine_mx_hidden_bytes(int k, int D, int F) {
  return align256((size_t)k * ((F + 127) / 128) * PB_BYTES) + align256((size_t)(D / 128) * PB_BYTES);
}

// planes_ready: x's plane blocks are already at xplanes (written by the router launch).
int launch_affine_mx(const uint16_t* x, bool planes_ready, uint8_t* hid, uint8_t* xplanes, const uint8_t* pool,
                     const Layout& L, const ExpertSource& src, int32_t* ws_slots, float* ws_w, int D, int F, int k,
                     int bits, int group, float limit, const uint16_t* addend, float* routed, uint16_t* out,
                     hipStream_t s) {
  if (!planes_ready)
    if (int rc = launch_x_planes(x, D, xplanes, s)) return rc;
#define CACHALOT_AMX(B, GG)                                                                                   \
  if (bits == B && group == GG)                                                                               \
    return launch_pair<B, GG>(xplanes, pool, L, src, ws_slots, ws_w, D, F, k, limit, addend, routed, out, hid, s);
  CACHALOT_AMX(2, 32) CACHALOT_AMX(2, 64)
  CACHALOT_AMX(3, 32) CACHALOT_AMX(3, 64) CACHALOT_AMX(3, 128)
  CACHALOT_AMX(4, 32) CACHALOT_AMX(4, 64) CACHALOT_AMX(4, 128)
#undef CACHALOT_AMX
  return fail(CACHALOT_EINVAL, "affine decode (matrix cores): %d-bit codes in groups of %d", bits, group);
}

}  // namespace cachalot
