// Decode (one token) over a 2-bit affine g128 bank in two launches on the
// block-scaled fp8 x fp4 matrix cores (mx_tile.h): v_mfma_scale_f32_16x16x128
// takes 16 weight rows x 128 codes per instruction, four times the weights of
// a bf16 step, with the 2-bit codes used as fp4 operands unconverted.
//
// Reference semantics: src/cachalot/model/expert_affine.py:65-81 (bf16 g, u,
// h, y_e rounding points), :117-152 (experts summed in route order from zero),
// mx.quantized_matmul's group formula s * sum(x q) + b * sum(x) (as copied at
// minimax/codes_qmv.py:86-100).
//
//   q2mx_gate_up_kernel  one 256-thread workgroup = one expert x one 16-row tile
//     of W1 and W3.  One wave (blockIdx % 4, so the routing waves of the
//     workgroups sharing a CU sit on different SIMDs) resolves the expert --
//     with the router's scores it runs the top-k itself -- while the other
//     three copy x's fp8 plane blocks (written once per token by the router
//     kernel or x_planes_kernel) into LDS.  Items are (tile, quad of four
//     128-code groups), quad q to wave q % 4.  Wave w copies the tile's run of
//     scale / bias tensor w into LDS (16 rows, whole lines), then loads its items'
//     codes; per item four block-scaled MFMAs per matrix sharing the A operand.  Epilogue: bf16(g), bf16(u), clamp,
//     h = bf16(silu(g) * u * w_e), stored as one fp8 plane piece of the
//     expert's hidden plane blocks (16 rows = one piece).
//   q2mx_down_kernel  one 768-thread workgroup = one 16-row tile of W2 for all k
//     experts; items (expert, quad) dealt round-robin to 12 waves.  The k
//     hidden plane blocks and the tile's scale / bias runs are copied into LDS;
//     each expert's row value is rounded to bf16 and the experts are summed in
//     route order, + addend.
//
// Summation orders (fixed, so results are reproducible): per item the four
// (piece, plane) partial sums of a group, then the four groups of a quad
// (lane-group butterfly), then the quads in order.
#include "decode_common.h"
#include "fp8_common.h"
#include "mfma_tile.h"
#include "mx_tile.h"
#include "permute_small.h"

namespace cachalot {
namespace {

using namespace decode;
using mx::a_role;
using mx::ARole;
using mx::bf16_lo;
using mx::Chain;
using mx::chain_init;
using mx::chain_load;
using mx::dot4;
using mx::f32x4_t;
using mx::i32x8_t;
using mx::PB_BYTES;
using mx::PB_SCALE;
using mx::PB_SUM;
using mx::piece_sums;

constexpr int GU_THREADS = 256;
constexpr int GU_WAVES = GU_THREADS / 64;
constexpr int MAX_GT = 40;                     // D <= 5120
constexpr int MAX_NQ = MAX_GT / 4;
constexpr int MAX_GK = 24;                     // F <= 3072
constexpr int MAX_NQ2 = MAX_GK / 4;
constexpr int DN_THREADS = 768;
constexpr int DN_WAVES = DN_THREADS / 64;

struct GuLds {
  uint8_t planes[MAX_GT * PB_BYTES];
  uint16_t sc[4][1024];   // s1, b1, s3, b3 of the tile's 16 rows (one run of 32 GT bytes each; 2 KiB slots)
  float red[MAX_NQ][2][16];
  int top_i[KMAX], top_s[KMAX];
  float top_v[KMAX], top_w[KMAX];
  int slot;
  float wexp;
};

struct DnLds {
  uint8_t planes[KMAX * MAX_GK * PB_BYTES];
  uint16_t sc[KMAX][2][512];              // per expert: s2, b2 runs of the tile's rows (32 GK bytes in a
                                          // 1 KiB slot: every lane of the copy writes its 16 bytes)
  float red[KMAX][MAX_NQ2][16];
  float y[KMAX][16];
};

using tile::copy_to_lds_untracked;

// x (one token) as fp8 plane blocks, for calls whose experts are given (no router launch).
__global__ void __launch_bounds__(256) x_planes_kernel(const uint16_t* __restrict__ x, int D,
                                                       uint8_t* __restrict__ xplanes) {
  const int t4 = blockIdx.x * 256 + threadIdx.x;
  if (4 * t4 < D) mx::encode_x_quad(xplanes, t4, reinterpret_cast<const uint2*>(x)[t4]);   // whole quads
}

// Workgroup bid of the gate/up grid (k * F / 16).  MAXM = ceil(D / 512 / 4) items per wave.
template <int MAXM>
__device__ __forceinline__ void q2mx_gate_up_body(GuLds& s, const int bid, const uint8_t* __restrict__ xplanes,
                                                  const uint8_t* __restrict__ pool, const Layout& L,
                                                  const ExpertSource& src, int D, int F, float limit,
                                                  uint8_t* __restrict__ hid, int32_t* __restrict__ ws_slots,
                                                  float* __restrict__ ws_w) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int GT = D / 128, NQ = GT / 4;
  const int GK = (F + 127) / 128, FT = F / 16;
  const int e = bid / FT;
  const int tile = bid - e * FT;
  const int row0 = tile * 16;
  const int rw = bid & (GU_WAVES - 1);   // the routing wave

  // ---- 0. routing wave: the expert's slot; the others: x's plane blocks into LDS
  if (wave == rw) {
    const int slot = route_slot(src, ws_slots, e, s.top_i, s.top_v, s.top_s);
    if (lane == 0) s.slot = slot;
    // (nothing is in flight here; the explicit wait tells the compiler so, and it then
    // puts no wait between the loads below)
    tile::wait_vmem();
  } else {
    copy_to_lds_untracked(xplanes, s.planes, GT * PB_BYTES, wave < rw ? wave : wave - 1, GU_WAVES - 1, lane);
    tile::wait_vmem();
  }
  lds_sync();
  // uniform (one value per workgroup): the loads below then take a scalar base and a
  // 32-bit vector offset, so no 64-bit address pair per load stays live
  const int slot = __builtin_amdgcn_readfirstlane(s.slot);
  const bool live = slot >= 0;

  // (set up before the loads, so these registers are not taken from the loads' addresses)
  const ARole ro = a_role(lane);
  Chain ch;
  chain_init(ch);

  // ---- 1. loads: wave w copies the tile's run of scale / bias tensor w (whole
  //         lines), then its items' codes; the runs are shared after a barrier
  uint4 c1[MAXM][2], c3[MAXM][2];
  if (live) {
    const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
    const int64_t toff = wave == 0 ? L.off[1] : wave == 1 ? L.off[2] : wave == 2 ? L.off[7] : L.off[8];
    // 32 GT bytes (<= 1280): one 1 KiB load, a second one (clamped source) past 32
    // columns; unpredicated, so that no wait lands between them and the codes
    const uint8_t* run = base + toff + (int64_t)row0 * GT * 2;
    uint8_t* dst = reinterpret_cast<uint8_t*>(s.sc[wave]);
    __builtin_amdgcn_global_load_lds(run + min(16 * lane, 32 * GT - 16), dst, 16, 0, 0);
    if (GT > 32) __builtin_amdgcn_global_load_lds(run + min(1024 + 16 * lane, 32 * GT - 16), dst + 1024, 16, 0, 0);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int q = min(wave + GU_WAVES * m, NQ - 1);
      const int off = (row0 + j) * (D / 4) + (4 * q + kg) * 32;   // < 2^31: a 16-row tile of one tensor
      const uint4* r1 = reinterpret_cast<const uint4*>(base + L.off[0] + off);
      const uint4* r3 = reinterpret_cast<const uint4*>(base + L.off[6] + off);
      c1[m][0] = r1[0];
      c1[m][1] = r1[1];
      c3[m][0] = r3[0];
      c3[m][1] = r3[1];
    }
  }
  // with scores, the routing wave normalises the selected weights while the loads
  // are in flight
  if (src.scores != nullptr && wave == rw) {
    const float w = route_weight(src, ws_w, e, s.top_v, s.top_w);
    if (lane == 0) s.wexp = w;
  }
  // the run copy, issued before the 4 * MAXM code loads, has landed (loads
  // complete in issue order); the codes stay in flight across the barrier
  if (live) __builtin_amdgcn_s_waitcnt(0x0F70 | (4 * MAXM));
  lds_sync();

  // ---- 2. items
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    const int q = wave + GU_WAVES * m;
    if (!live || q >= NQ) break;
    f32x4_t a1 = mx::zero_acc(), a3 = mx::zero_acc();
    chain_load(ch, s.planes + (4 * q + ro.kgR) * PB_BYTES, ro);
    a1 = mx::mfma_fp8_fp4<0>(ch.a[0], mx::q2_spread(c1[m][0].x, c1[m][0].y), a1, ch.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<0>(ch.a[0], mx::q2_spread(c3[m][0].x, c3[m][0].y), a3, ch.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<1>(ch.a[1], mx::q2_spread(c1[m][0].z, c1[m][0].w), a1, ch.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<1>(ch.a[1], mx::q2_spread(c3[m][0].z, c3[m][0].w), a3, ch.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<2>(ch.a[2], mx::q2_spread(c1[m][1].x, c1[m][1].y), a1, ch.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<2>(ch.a[2], mx::q2_spread(c3[m][1].x, c3[m][1].y), a3, ch.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<3>(ch.a[3], mx::q2_spread(c1[m][1].z, c1[m][1].w), a1, ch.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<3>(ch.a[3], mx::q2_spread(c3[m][1].z, c3[m][1].w), a3, ch.sa, mx::E8M0_TWO);
    const float sx = piece_sums(s.planes + (4 * q + kg) * PB_BYTES, mx::PIECES);
    const int si = j * GT + 4 * q + kg;
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
    // the expert's slot for the down kernel, stored here rather than before the loads:
    // a store's data registers stay busy until it completes (one counter on gfx9)
    if (tid == 0 && (src.idx || src.scores) && tile == 0) ws_slots[e] = slot;
    // given experts: the weight is loaded here (measured faster than with the slot)
    const float wexp = src.scores != nullptr ? s.wexp : expert_weight(src, ws_w, e);
    if (src.scores != nullptr) {   // the selection, for the down kernel and the caller
      if (tile == 0 && tid == 0) ws_w[e] = wexp;
      if (bid == 0 && tid < src.k) {
        if (src.idx_out) src.idx_out[tid] = s.top_i[tid];
        if (src.w_out) src.w_out[tid] = s.top_w[tid];
      }
    }
    float hv = 0.0f;
    if (live) {
      float rg[MAX_NQ], ru[MAX_NQ];
#pragma unroll
      for (int q = 0; q < MAX_NQ; ++q) {
        rg[q] = s.red[q][0][tid];
        ru[q] = s.red[q][1][tid];
      }
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int q = 0; q < MAX_NQ; ++q) {
        if (q < NQ) {
          g = g + rg[q];
          u = u + ru[q];
        }
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
    if (tile == FT - 1) {   // pieces of the last group past F: zeros (consumers read whole steps)
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

template <int MAXM>
__global__ void __launch_bounds__(GU_THREADS) q2mx_gate_up_kernel(const uint8_t* __restrict__ xplanes,
                                                                  const uint8_t* __restrict__ pool, Layout L,
                                                                  ExpertSource src, int D, int F, float limit,
                                                                  uint8_t* __restrict__ hid,
                                                                  int32_t* __restrict__ ws_slots,
                                                                  float* __restrict__ ws_w) {
  __shared__ __align__(16) GuLds s;
  q2mx_gate_up_body<MAXM>(s, blockIdx.x, xplanes, pool, L, src, D, F, limit, hid, ws_slots, ws_w);
}

using fp8::SH_CPV;
using fp8::SH_MAX_K;

// grid.x = k * F / 16 + n_sh: the routed workgroups, then the shared expert's gate/up
// tiles.  (Workgroups are dispatched in order and not all of them fit the chip at
// once: the shared tiles, which need no routing, go last, into the slots the first
// routed workgroups leave; measured 36.3 us per layer with them first, 34.9
// interleaved one in four, 33.7 last.)
template <int MAXM>
__global__ void __launch_bounds__(GU_THREADS) q2mx_gate_up_shared_kernel(const uint8_t* __restrict__ xplanes,
                                                                         const uint8_t* __restrict__ pool, Layout L,
                                                                         ExpertSource src, int D, int F, float limit,
                                                                         uint8_t* __restrict__ hid,
                                                                         int32_t* __restrict__ ws_slots,
                                                                         float* __restrict__ ws_w,
                                                                         fp8::DecodeArgs sh, int n_sh) {
  constexpr int SH_LDS = fp8::dec_tile_lds(1, SH_MAX_K);
  __shared__ __align__(16) uint8_t buf[sizeof(GuLds) > SH_LDS ? sizeof(GuLds) : SH_LDS];
  if ((int)blockIdx.x >= (int)gridDim.x - n_sh) {
    fp8::shared_gu_tile<GU_THREADS>(sh, blockIdx.x - (gridDim.x - n_sh), buf);
    return;
  }
  q2mx_gate_up_body<MAXM>(*reinterpret_cast<GuLds*>(buf), blockIdx.x, xplanes, pool, L, src, D, F, limit,
                          hid, ws_slots, ws_w);
}

// Down items m0 .. m0 + NI - 1 of a wave, interleaved.
template <int NI, int MAXM>
__device__ __forceinline__ void down_items(DnLds& s, const uint4 (&c2)[MAXM][2], const int (&it_e)[MAXM],
                                           const int (&it_q)[MAXM], const bool (&on)[MAXM], int m0,
                                           const ARole& ro, int GK, int FT, int j, int kg, int lane, bool f16) {
  Chain ch[NI];
  f32x4_t acc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int m = m0 + i;
    chain_init(ch[i]);
    chain_load(ch[i], s.planes + (it_e[m] * GK + min(4 * it_q[m] + ro.kgR, GK - 1)) * PB_BYTES, ro);
    acc[i] = mx::zero_acc();
  }
#pragma unroll
  for (int i = 0; i < NI; ++i)
    acc[i] = mx::mfma_fp8_fp4<0>(ch[i].a[0], mx::q2_spread(c2[m0 + i][0].x, c2[m0 + i][0].y), acc[i], ch[i].sa,
                                 mx::E8M0_TWO);
#pragma unroll
  for (int i = 0; i < NI; ++i)
    acc[i] = mx::mfma_fp8_fp4<1>(ch[i].a[1], mx::q2_spread(c2[m0 + i][0].z, c2[m0 + i][0].w), acc[i], ch[i].sa,
                                 mx::E8M0_TWO);
#pragma unroll
  for (int i = 0; i < NI; ++i)
    acc[i] = mx::mfma_fp8_fp4<2>(ch[i].a[2], mx::q2_spread(c2[m0 + i][1].x, c2[m0 + i][1].y), acc[i], ch[i].sa,
                                 mx::E8M0_TWO);
#pragma unroll
  for (int i = 0; i < NI; ++i)
    acc[i] = mx::mfma_fp8_fp4<3>(ch[i].a[3], mx::q2_spread(c2[m0 + i][1].z, c2[m0 + i][1].w), acc[i], ch[i].sa,
                                 mx::E8M0_TWO);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int m = m0 + i;
    const int e = it_e[m], q2 = it_q[m];
    const int g2 = 4 * q2 + kg;
    const float sh = g2 < GK ? piece_sums(s.planes + (e * GK + g2) * PB_BYTES, min(8, FT - 8 * g2)) : 0.0f;
    const int si = j * GK + min(g2, GK - 1);
    float v = g2 < GK ? scale_bits_to_f32(s.sc[e][0][si], f16) * dot4(acc[i]) + scale_bits_to_f32(s.sc[e][1][si], f16) * sh
                      : 0.0f;
    v = tile::sum_lane_groups(v);
    if (on[m] && lane < 16) s.red[e][q2][lane] = v;
  }
}

// grid.x = D / 16.  MAXM = ceil(k * ceil(GK / 4) / 12) items per wave.  SH: the
// workgroup also runs the shared expert's down tile of the same 16 rows (w2 over
// act_quant(h_sh), sh.a = h_sh), whose bf16 y is the addend.
template <int MAXM, bool SH>
__global__ void __launch_bounds__(DN_THREADS) q2mx_down_kernel(const uint8_t* __restrict__ pool, Layout L,
                                                               const int32_t* __restrict__ ws_slots, int D, int F,
                                                               int k, const uint8_t* __restrict__ hid,
                                                               const uint16_t* __restrict__ addend,
                                                               float* __restrict__ routed,
                                                               uint16_t* __restrict__ out, fp8::DecodeArgs sh) {
  __shared__ __align__(16) DnLds s;
  // shared expert: act_quant(h_sh) and the partial tiles, its 16 w2 rows (16 K bytes),
  // h_sh as copied (bf16) and the tile's scale row
  constexpr int SH_TILE = fp8::dec_tile_lds(1, SH_MAX_K);
  __shared__ __align__(16) uint8_t sh_lds[SH ? SH_TILE + 18 * SH_MAX_K + SH_MAX_K / 32 : 16];
  constexpr int SH_NPV = (fp8::DEC_VW + DN_WAVES - 1) / DN_WAVES;   // virtual waves per wave (2)
  uint8_t* sh_w = sh_lds + SH_TILE;
  uint8_t* sh_h = sh_w + 16 * SH_MAX_K;
  uint8_t* sh_sc = sh_h + 2 * SH_MAX_K;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int GK = (F + 127) / 128, NQ2 = (GK + 3) / 4, FT = F / 16;
  const int row0 = blockIdx.x * 16;
  const int n_items = k * NQ2;

  // ---- 0. the hidden plane blocks into LDS; the slots (KMAX entries are
  //         allocated) -> the tile's scale / bias runs into LDS, then the wave's
  //         W2 codes into registers
  // (the shared expert's scale row first: one byte per thread, into LDS at the barrier)
  uint32_t sh_sb = 0;
  if constexpr (SH) sh_sb = sh.ws[0][(size_t)(row0 / 32) * (sh.K / 32) + min(tid, sh.K / 32 - 1)];
  // the hidden plane blocks first: they do not wait for the slots
  copy_to_lds_untracked(hid, s.planes, k * GK * PB_BYTES, wave, DN_WAVES, lane);
  // the shared expert's h (bf16; its 16 w2 rows follow the routed codes)
  if constexpr (SH)
    copy_to_lds_untracked(reinterpret_cast<const uint8_t*>(sh.a), sh_h, 2 * sh.K, wave, DN_WAVES, lane);
  // the tile's addend, read now rather than in the epilogue (every lane loads, no
  // branch: the wait for it then sits at its use)
  const uint16_t add_bits = (addend != nullptr ? addend : reinterpret_cast<const uint16_t*>(hid))[row0 + (tid & 15)];
  int eslot[KMAX];
#pragma unroll
  for (int e = 0; e < KMAX; ++e) eslot[e] = ws_slots[e];
  {
    // the tile's scale / bias runs (one per wave: 32 GK <= 1 KiB), before the codes
    const int run = 32 * GK;   // 16 rows x GK bf16
#pragma unroll
    for (int r0 = 0; r0 < 2 * KMAX; r0 += DN_WAVES) {
      const int r = r0 + wave;
      if (r < 2 * k) {
        int ps = eslot[0];
#pragma unroll
        for (int e = 1; e < KMAX; ++e) ps = e == (r >> 1) ? eslot[e] : ps;
        ps = max(ps, 0);   // a missing expert's rows are never used
        const uint8_t* src = pool + (int64_t)ps * L.record_bytes + ((r & 1) ? L.off[5] : L.off[4]) +
                             (int64_t)row0 * GK * 2;
        tile::lds_load16_untracked(src + min(16 * lane, run - 16), reinterpret_cast<uint8_t*>(s.sc[r >> 1][r & 1]));
      }
    }
  }
  uint4 c2[MAXM][2];
  int it_e[MAXM], it_q[MAXM];
  bool on[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    const int it = wave + DN_WAVES * m;
    const int itc = min(it, n_items - 1);
    it_e[m] = itc / NQ2;
    it_q[m] = itc - it_e[m] * NQ2;
    int slot = eslot[0];
#pragma unroll
    for (int e = 1; e < KMAX; ++e) slot = e == it_e[m] ? eslot[e] : slot;
    on[m] = it < n_items && slot >= 0;
    const int g2 = min(4 * it_q[m] + kg, GK - 1);
    const uint8_t* base = pool + (int64_t)max(slot, 0) * L.record_bytes;
    const uint4* r2 = reinterpret_cast<const uint4*>(base + L.off[3] + (int64_t)(row0 + j) * (GK * 32) + g2 * 32);
    c2[m][0] = r2[0];
    c2[m][1] = r2[1];
  }
  // the copies, issued before the 2 MAXM code loads, have landed (loads complete in
  // issue order); the codes stay in flight, each item waits for its own
  __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * MAXM));
  // then the shared expert's 16 w2 rows (contiguous, 16 K bytes), in flight during
  // the items and waited for after them
  if constexpr (SH) copy_to_lds_untracked(sh.w[0] + (size_t)row0 * sh.K, sh_w, 16 * sh.K, wave, DN_WAVES, lane);
  if (SH && tid < sh.K / 32) sh_sc[tid] = (uint8_t)sh_sb;
  lds_sync();
  if constexpr (SH) {   // act_quant(h_sh) into LDS, read after the items' barrier
    fp8::DecAct<1, DN_THREADS> xa;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(xa.v) / sizeof(xa.v[0])); ++i)
      xa.v[i] = *reinterpret_cast<const uint4*>(sh_h + 16 * min(tid + DN_THREADS * i, sh.K / 8 - 1));
    fp8::dec_act_quant<1, DN_THREADS>(sh, 1, tid, xa, sh_lds);
  }

  // ---- 1. items, in interleaved groups (every item's A operands, then each MFMA step
  //         for all items of the group: independent accumulators keep the matrix
  //         pipeline busy), then the group formulas.  Items that are off compute on
  //         valid (clamped) data and are discarded.
  const ARole ro = a_role(lane);
  if constexpr (MAXM <= 3) {
    down_items<MAXM>(s, c2, it_e, it_q, on, 0, ro, GK, FT, j, kg, lane, L.f16);
  } else {
    down_items<2>(s, c2, it_e, it_q, on, 0, ro, GK, FT, j, kg, lane, L.f16);
    down_items<MAXM - 2>(s, c2, it_e, it_q, on, 2, ro, GK, FT, j, kg, lane, L.f16);
  }
  if constexpr (SH) tile::wait_vmem();   // the shared rows
  lds_sync();
  if constexpr (SH) {   // the shared tile's partial tiles (read after the next barrier)
    uint32_t bs[SH_NPV][SH_CPV];
    fp8::dec_wscale<SH_NPV, SH_CPV>(sh_sc, sh.K, wave, DN_WAVES, lane, bs);
    fp8::dec_mfma_wlds<1, SH_NPV, SH_CPV>(sh, 1, wave, DN_WAVES, lane, sh_w, bs, sh_lds);
  }

  // ---- 2. per expert (16 lanes each): the row values rounded to bf16; then the
  //         route-order sum of the tile's rows
  if (tid < 16 * k) {
    const int e = tid >> 4, r = tid & 15;
    float part[MAX_NQ2];
#pragma unroll
    for (int q2 = 0; q2 < MAX_NQ2; ++q2) part[q2] = s.red[e][q2][r];
    float y = 0.0f;
#pragma unroll
    for (int q2 = 0; q2 < MAX_NQ2; ++q2)
      if (q2 < NQ2) y = y + part[q2];
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
    if constexpr (SH) {
      if (out) out[n] = f32_to_bf16(total + round_bf16(fp8::dec_total(sh_lds, 1, sh.K, tid, 0)));
    } else {
      if (out) out[n] = f32_to_bf16(addend ? total + bf16_to_f32(add_bits) : total);
    }
  }
}

// ------------------------------------------------------ batched (expert-major) ---
// Few tokens per expert (batched decode, speculative verify): the rows of one expert
// (permuted expert-major, grouped.hip) share one load of its codes.  The same tiles,
// items and arithmetic as the one-token kernels above, run once per row with that
// row's activation planes; the next row's planes are copied into LDS while the
// current row computes.
//   q2mx_bgu_kernel   grid (F / 16, active experts): h planes of every row, [rows][GK]
//   q2mx_bdn4_kernel  grid (D / 64, active experts): y = bf16(h W2) of every row, to
//                     its (token, route slot) place of y [T, k, D]
// Tiles run along grid.x, experts along grid.y: workgroups are dispatched x-first, so
// the workgroups in flight read neighbouring tiles of few experts -- long contiguous
// runs of the bank -- rather than one tile of every expert (measured at B = 32: gate/up
// 266 -> 216 us, down 160 -> 128 us).
struct BatchArgs {
  const uint8_t* xplanes;   // [T][D / 128] plane blocks
  const uint8_t* pool;
  Layout L;
  const int4* recs;         // (expert, first row, end row, slot) of every expert with rows
  const int32_t* n_recs;
  const int32_t* row_token;
  const int32_t* row_slot;
  const float* row_w;
  int D, F, k;
  float limit;
  uint8_t* hid;             // [rows][GK] plane blocks
  uint16_t* y;              // [T, k, D]
};

// sized for D <= 2048 * MAXM, so that more workgroups fit a CU at the smaller widths
template <int MAXM>
struct BGuLds {
  uint8_t planes[2][4 * GU_WAVES * MAXM * PB_BYTES];
  uint16_t sc[4][16 * MAX_GT];   // s1, b1, s3, b3 of the tile's 16 rows (one contiguous run each)
  float red[GU_WAVES * MAXM][2][16];
};

// One launch before the batched kernels, grid 2 + T * ceil(D / 4096), 1024 threads:
//   workgroup 0: the record (expert, first row, end row, slot) of every expert with
//     rows, experts ascending, and their count -- so a batched workgroup reads one
//     record and issues its weight loads, with no dependent lookup in between;
//   the last: zero y rows of the dropped routes (rows [offsets[E], n) of the
//     permutation; entries outside [0, T) x [0, k) skipped), so the combine adds
//     nothing for them -- the batched path's own copy of the grouped drop pass;
//   the others: x (T tokens) as plane blocks, 1024 quads each.
constexpr int PREP_THREADS = 1024;
// The dropped routes' y rows (rows [offsets[E], n) of the permutation) cleared by
// one workgroup.
__device__ __forceinline__ void clear_dropped_rows(const int32_t* offsets, int E, int n, int T, int k, int D,
                                                   const int32_t* row_token, const int32_t* row_slot, uint16_t* y) {
  const int first = offsets[E];
  const int per_row = D / 8;   // 16-byte stores
  const int total = max(n - first, 0) * per_row;
  for (int i = threadIdx.x; i < total; i += PREP_THREADS) {
    const int r = first + i / per_row;
    const int c = i - (r - first) * per_row;
    const int t = row_token[r], sl = row_slot[r];
    if (t < 0 || t >= T || sl < 0 || sl >= k) continue;
    reinterpret_cast<uint4*>(y + ((size_t)t * k + sl) * D)[c] = uint4{0u, 0u, 0u, 0u};
  }
}

// ridx / rw (the routes [n], or null when the caller permuted them): workgroup 0
// first runs the permutation itself (permute_small_body, n <= PREP_THREADS) and, after
// the records, clears the dropped routes' rows; without routes the last workgroup
// of the grid clears them.
__global__ void __launch_bounds__(PREP_THREADS) batch_prep_kernel(const uint16_t* __restrict__ x, int T, int D,
                                                                  uint8_t* __restrict__ xplanes,
                                                                  int32_t* __restrict__ offsets, int E,
                                                                  const int32_t* __restrict__ slot_table,
                                                                  int4* __restrict__ recs, int32_t* __restrict__ n_recs,
                                                                  int n, int k, int32_t* __restrict__ row_token,
                                                                  int32_t* __restrict__ row_slot,
                                                                  uint16_t* __restrict__ y,
                                                                  const int32_t* __restrict__ ridx,
                                                                  const float* __restrict__ rw,
                                                                  float* __restrict__ row_w) {
  const int tid = threadIdx.x;
  if (ridx == nullptr && blockIdx.x == gridDim.x - 1) {
    clear_dropped_rows(offsets, E, n, T, k, D, row_token, row_slot, y);
    return;
  }
  if (blockIdx.x > 0) {
    const int per_row = (D + 4095) / 4096;
    const int t = (blockIdx.x - 1) / per_row;
    const int t4 = ((blockIdx.x - 1) - t * per_row) * PREP_THREADS + tid;
    if (4 * t4 < D)
      mx::encode_x_quad(xplanes + (size_t)t * (D / 128) * PB_BYTES, t4,
                        reinterpret_cast<const uint2*>(x + (size_t)t * D)[t4]);   // whole quads
    return;
  }
  if (ridx != nullptr) {
    permute_small_body<PREP_THREADS>(ridx, rw, n, k, E, offsets, row_token, row_slot, row_w);
    __syncthreads();   // the offsets and rows are this workgroup's own global stores
  }
  __shared__ int wave_n[PREP_THREADS / 64];
  const int lane = tid & 63, wave = tid >> 6;
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += PREP_THREADS) {   // E <= 1024: one trip
    const int e = e0 + tid;
    int r0 = 0, r1 = 0;
    if (e < E) {
      r0 = offsets[e];
      r1 = offsets[e + 1];
    }
    const bool active = r1 > r0;
    const uint64_t m = __ballot(active);
    if (lane == 0) wave_n[wave] = __popcll(m);
    __syncthreads();
    int before = base, total = base;
    for (int w = 0; w < PREP_THREADS / 64; ++w) {
      before += w < wave ? wave_n[w] : 0;
      total += wave_n[w];
    }
    if (active) recs[before + __popcll(m & ((1ull << lane) - 1ull))] = make_int4(e, r0, r1, slot_table[e]);
    base = total;
    __syncthreads();
  }
  if (tid == 0) n_recs[0] = base;
  if (ridx != nullptr) clear_dropped_rows(offsets, E, n, T, k, D, row_token, row_slot, y);
}

template <int MAXM>
__global__ void __launch_bounds__(GU_THREADS) q2mx_bgu_kernel(BatchArgs a) {
  __shared__ __align__(16) BGuLds<MAXM> s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  // the record and the count load together (grid.x = the records allocated)
  const int4 rec = a.recs[blockIdx.y];
  if ((int)blockIdx.y >= a.n_recs[0]) return;
  const int r0 = __builtin_amdgcn_readfirstlane(rec.y);
  const int r1 = __builtin_amdgcn_readfirstlane(rec.z);
  const int slot = __builtin_amdgcn_readfirstlane(rec.w);
  const int D = a.D, F = a.F;
  const int GT = D / 128, NQ = GT / 4;
  const int GK = (F + 127) / 128, FT = F / 16;
  const int tile = blockIdx.x;
  const int row0 = tile * 16;
  const bool live = slot >= 0;
  const int pbytes = GT * PB_BYTES;

  // the first row's planes, then the tile's scale chunks and codes
  copy_to_lds_untracked(a.xplanes + (size_t)a.row_token[r0] * pbytes, s.planes[0], pbytes, wave, GU_WAVES, lane);
  // (unconditional: a missing expert reads slot 0's bytes and discards them, so the
  // code registers are defined on one path and the compiler copies none of them)
  uint4 c1[MAXM][2], c3[MAXM][2];
  {
    const uint8_t* base = a.pool + (int64_t)max(slot, 0) * a.L.record_bytes;
    // wave w: the 16 rows' run of scale / bias tensor w (whole lines)
    const int64_t toff = wave == 0 ? a.L.off[1] : wave == 1 ? a.L.off[2] : wave == 2 ? a.L.off[7] : a.L.off[8];
    copy_to_lds_untracked(base + toff + (int64_t)row0 * GT * 2, reinterpret_cast<uint8_t*>(s.sc[wave]), 32 * GT, 0,
                          1, lane);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int q = min(wave + GU_WAVES * m, NQ - 1);
      const int64_t off = (int64_t)(row0 + j) * (D / 4) + (4 * q + kg) * 32;
      const uint4* w1 = reinterpret_cast<const uint4*>(base + a.L.off[0] + off);
      const uint4* w3 = reinterpret_cast<const uint4*>(base + a.L.off[6] + off);
      c1[m][0] = w1[0];
      c1[m][1] = w1[1];
      c3[m][0] = w3[0];
      c3[m][1] = w3[1];
    }
  }
  // the copies (issued first) have landed; the codes stay in flight, each item waits
  // for its own
  __builtin_amdgcn_s_waitcnt(0x0F70 | (4 * MAXM));
  lds_sync();
  const ARole ro = a_role(lane);
  Chain ch;
  chain_init(ch);
  for (int r = r0; r < r1; ++r) {
    const int buf = __builtin_amdgcn_readfirstlane((r - r0) & 1);
    // the next row's planes, into the other buffer, by waves 1.. (wave 0 stores this
    // row's h below and then need not wait for its own stores)
    if (r + 1 < r1 && wave > 0)
      copy_to_lds_untracked(a.xplanes + (size_t)a.row_token[r + 1] * pbytes, s.planes[buf ^ 1], pbytes, wave - 1,
                            GU_WAVES - 1, lane);
    const uint8_t* planes = s.planes[buf];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int q = wave + GU_WAVES * m;
      if (!live || q >= NQ) break;
      // items in order, each waiting only for its own codes (the asm pins the codes'
      // first use here, so their conversion is not hoisted above the earlier items)
      asm volatile("" : "+v"(c1[m][0].x), "+v"(c1[m][0].y), "+v"(c1[m][0].z), "+v"(c1[m][0].w),
                   "+v"(c1[m][1].x), "+v"(c1[m][1].y), "+v"(c1[m][1].z), "+v"(c1[m][1].w)::"memory");
      asm volatile("" : "+v"(c3[m][0].x), "+v"(c3[m][0].y), "+v"(c3[m][0].z), "+v"(c3[m][0].w),
                   "+v"(c3[m][1].x), "+v"(c3[m][1].y), "+v"(c3[m][1].z), "+v"(c3[m][1].w)::"memory");
      f32x4_t a1 = mx::zero_acc(), a3 = mx::zero_acc();
      chain_load(ch, planes + (4 * q + ro.kgR) * PB_BYTES, ro);
      a1 = mx::mfma_fp8_fp4<0>(ch.a[0], mx::q2_spread(c1[m][0].x, c1[m][0].y), a1, ch.sa, mx::E8M0_TWO);
      a3 = mx::mfma_fp8_fp4<0>(ch.a[0], mx::q2_spread(c3[m][0].x, c3[m][0].y), a3, ch.sa, mx::E8M0_TWO);
      a1 = mx::mfma_fp8_fp4<1>(ch.a[1], mx::q2_spread(c1[m][0].z, c1[m][0].w), a1, ch.sa, mx::E8M0_TWO);
      a3 = mx::mfma_fp8_fp4<1>(ch.a[1], mx::q2_spread(c3[m][0].z, c3[m][0].w), a3, ch.sa, mx::E8M0_TWO);
      a1 = mx::mfma_fp8_fp4<2>(ch.a[2], mx::q2_spread(c1[m][1].x, c1[m][1].y), a1, ch.sa, mx::E8M0_TWO);
      a3 = mx::mfma_fp8_fp4<2>(ch.a[2], mx::q2_spread(c3[m][1].x, c3[m][1].y), a3, ch.sa, mx::E8M0_TWO);
      a1 = mx::mfma_fp8_fp4<3>(ch.a[3], mx::q2_spread(c1[m][1].z, c1[m][1].w), a1, ch.sa, mx::E8M0_TWO);
      a3 = mx::mfma_fp8_fp4<3>(ch.a[3], mx::q2_spread(c3[m][1].z, c3[m][1].w), a3, ch.sa, mx::E8M0_TWO);
      const float sx = piece_sums(planes + (4 * q + kg) * PB_BYTES, mx::PIECES);
      const int si = j * GT + 4 * q + kg;
      const float v1 = scale_bits_to_f32(s.sc[0][si], a.L.f16) * dot4(a1) + scale_bits_to_f32(s.sc[1][si], a.L.f16) * sx;
      const float v3 = scale_bits_to_f32(s.sc[2][si], a.L.f16) * dot4(a3) + scale_bits_to_f32(s.sc[3][si], a.L.f16) * sx;
      const float s1 = tile::sum_lane_groups(v1);
      const float s3 = tile::sum_lane_groups(v3);
      if (lane < 16) {
        s.red[q][0][lane] = s1;
        s.red[q][1][lane] = s3;
      }
    }
    lds_sync();
    if (tid < 16) {
      float hv = 0.0f;
      if (live) {
        float rg[GU_WAVES * MAXM], ru[GU_WAVES * MAXM];
#pragma unroll
        for (int q = 0; q < GU_WAVES * MAXM; ++q) {
          rg[q] = s.red[q][0][tid];
          ru[q] = s.red[q][1][tid];
        }
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int q = 0; q < GU_WAVES * MAXM; ++q) {
          if (q < NQ) {
            g = g + rg[q];
            u = u + ru[q];
          }
        }
        g = round_bf16(g);
        u = round_bf16(u);
        if (a.limit > 0.0f) {
          u = fminf(fmaxf(u, -a.limit), a.limit);
          g = fminf(g, a.limit);
        }
        hv = round_bf16((silu_f32(g) * u) * a.row_w[r]);
      }
      const mx::PieceCode pc = mx::encode_piece(hv);
      const int pp = tile & 7;
      uint8_t* blk = a.hid + ((int64_t)r * GK + (tile >> 3)) * PB_BYTES;
      blk[mx::pb_data(pp, 0) + mx::piece_pos(tid)] = (uint8_t)pc.hi;
      blk[mx::pb_data(pp, 1) + mx::piece_pos(tid)] = (uint8_t)pc.lo;
      if (tid == 0) {
        blk[mx::pb_scale(pp, 0)] = (uint8_t)pc.scales;
        blk[mx::pb_scale(pp, 1)] = (uint8_t)(pc.scales >> 8);
        *reinterpret_cast<float*>(blk + PB_SUM + 4 * pp) = pc.sum;
      }
      if (tile == FT - 1) {
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
    // before the next row: its planes have landed (the copying waves' loads) and
    // every wave is past this row's reads of red and of the current planes.  After
    // the last row nothing waits, so the workgroup ends while its stores drain.
    if (r + 1 < r1) {
      if (wave > 0) tile::wait_vmem();
      lds_sync();
    }
  }
}

// Down over 64 output rows per workgroup: wave w owns the 16-row tile n0 + 16 w and
// all of its quads (items (expert, quad) as in q2mx_down_kernel), so a workgroup
// holds 4x the codes of a 16-row workgroup, and each row's sum over the quads stays
// in the wave, in quad order (the order of the one-token kernel's LDS reduction).
struct BDn4Lds {
  uint8_t planes[2][MAX_GK * PB_BYTES];
  uint16_t sc[GU_WAVES][2][16 * MAX_GK];   // per wave: s2, b2 runs of its rows
};

__global__ void __launch_bounds__(GU_THREADS) q2mx_bdn4_kernel(BatchArgs a) {
  __shared__ __align__(16) BDn4Lds s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kg = lane >> 4;
  const int4 rec = a.recs[blockIdx.y];
  if ((int)blockIdx.y >= a.n_recs[0]) return;
  const int r0 = __builtin_amdgcn_readfirstlane(rec.y);
  const int r1 = __builtin_amdgcn_readfirstlane(rec.z);
  const int slot = __builtin_amdgcn_readfirstlane(rec.w);
  const int D = a.D, F = a.F;
  const int GK = (F + 127) / 128, NQ2 = (GK + 3) / 4, FT = F / 16;
  const int n0 = blockIdx.x * 64 + wave * 16;
  const bool live = slot >= 0;
  const int hbytes = GK * PB_BYTES;

  copy_to_lds_untracked(a.hid + (size_t)r0 * hbytes, s.planes[0], hbytes, wave, GU_WAVES, lane);
  // (unconditional: a missing expert reads slot 0's bytes and discards them, so the
  // code registers are defined on one path and the compiler copies none of them)
  uint4 c2[MAX_NQ2][2];
  {
    const uint8_t* base = a.pool + (int64_t)max(slot, 0) * a.L.record_bytes;
    const int run = 32 * GK;
    copy_to_lds_untracked(base + a.L.off[4] + (int64_t)n0 * GK * 2, reinterpret_cast<uint8_t*>(s.sc[wave][0]), run,
                          0, 1, lane);
    copy_to_lds_untracked(base + a.L.off[5] + (int64_t)n0 * GK * 2, reinterpret_cast<uint8_t*>(s.sc[wave][1]), run,
                          0, 1, lane);
#pragma unroll
    for (int m = 0; m < MAX_NQ2; ++m) {
      const int g2 = min(4 * min(m, NQ2 - 1) + kg, GK - 1);
      const uint4* w2 = reinterpret_cast<const uint4*>(base + a.L.off[3] + (int64_t)(n0 + j) * (GK * 32) + g2 * 32);
      c2[m][0] = w2[0];
      c2[m][1] = w2[1];
    }
  }
  // the copies (issued first) have landed; the codes stay in flight, each item waits
  // for its own
  __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * MAX_NQ2));
  lds_sync();
  const ARole ro = a_role(lane);
  Chain ch;
  chain_init(ch);
  float ylast = 0.0f;
  int rlast = -1;
  for (int r = r0; r < r1; ++r) {
    const int buf = __builtin_amdgcn_readfirstlane((r - r0) & 1);
    if (r + 1 < r1)
      copy_to_lds_untracked(a.hid + (size_t)(r + 1) * hbytes, s.planes[buf ^ 1], hbytes, wave, GU_WAVES, lane);
    const uint8_t* planes = s.planes[buf];
    float yv = 0.0f;
#pragma unroll
    for (int m = 0; m < MAX_NQ2; ++m) {
      if (!live || m >= NQ2) break;
      // items in order, each waiting only for its own codes (the asm pins the codes'
      // first use here, so their conversion is not hoisted above the earlier items)
      asm volatile("" : "+v"(c2[m][0].x), "+v"(c2[m][0].y), "+v"(c2[m][0].z), "+v"(c2[m][0].w),
                   "+v"(c2[m][1].x), "+v"(c2[m][1].y), "+v"(c2[m][1].z), "+v"(c2[m][1].w)::"memory");
      const int g2 = 4 * m + kg;
      f32x4_t acc = mx::zero_acc();
      chain_load(ch, planes + min(4 * m + ro.kgR, GK - 1) * PB_BYTES, ro);
      acc = mx::mfma_fp8_fp4<0>(ch.a[0], mx::q2_spread(c2[m][0].x, c2[m][0].y), acc, ch.sa, mx::E8M0_TWO);
      acc = mx::mfma_fp8_fp4<1>(ch.a[1], mx::q2_spread(c2[m][0].z, c2[m][0].w), acc, ch.sa, mx::E8M0_TWO);
      acc = mx::mfma_fp8_fp4<2>(ch.a[2], mx::q2_spread(c2[m][1].x, c2[m][1].y), acc, ch.sa, mx::E8M0_TWO);
      acc = mx::mfma_fp8_fp4<3>(ch.a[3], mx::q2_spread(c2[m][1].z, c2[m][1].w), acc, ch.sa, mx::E8M0_TWO);
      const float sh = g2 < GK ? piece_sums(planes + g2 * PB_BYTES, min(8, FT - 8 * g2)) : 0.0f;
      const int si = j * GK + min(g2, GK - 1);
      float v = g2 < GK ? scale_bits_to_f32(s.sc[wave][0][si], a.L.f16) * dot4(acc) +
                              scale_bits_to_f32(s.sc[wave][1][si], a.L.f16) * sh
                        : 0.0f;
      yv = yv + tile::sum_lane_groups(v);
    }
    // the previous row's outputs go out now: their stores then overlap this row's work
    if (rlast >= 0 && lane < 16)
      a.y[((size_t)a.row_token[rlast] * a.k + a.row_slot[rlast]) * D + n0 + lane] = f32_to_bf16(ylast);
    ylast = yv;
    rlast = r;
    if (r + 1 < r1) {
      tile::wait_vmem();
      lds_sync();
    }
  }
  if (lane < 16) a.y[((size_t)a.row_token[rlast] * a.k + a.row_slot[rlast]) * D + n0 + lane] = f32_to_bf16(ylast);
}

}  // namespace

// x (one token) as plane blocks, for decode calls whose router launch did not write them.
int launch_x_planes(const uint16_t* x, int D, uint8_t* xplanes, hipStream_t s) {
  hipLaunchKernelGGL(x_planes_kernel, dim3((D / 4 + 255) / 256), dim3(256), 0, s, x, D, xplanes);
  return check_launch("x_planes_kernel");
}

// The shapes the matrix-core path takes (the rest use the bf16 kernels).
bool q2mx_supported(int D, int F, int k) {
  return D % 1024 == 0 && D <= 128 * MAX_GT && F % 16 == 0 && F <= 128 * MAX_GK && k >= 1 && k <= KMAX;
}

// The shapes the routed launches carry the shared expert for (else it runs in its
// own launches before them): one token, K <= SH_MAX_K on both sides.
bool q2mx_shared_supported(int D, int F_sh) { return D <= SH_MAX_K && F_sh <= SH_MAX_K; }

// hid: k * ceil(F / 128) plane blocks; xplanes: D / 128 plane blocks, written by
// the router kernel when planes_ready, else here.  sh_gu / sh_dn (both or neither):
// the shared expert's gate/up (out = h_sh [F_sh]) and down (a = h_sh) tiles, carried
// by the two routed launches; out then gets bf16(routed + y_sh) and addend is null.
int launch_q2mx_decode(const uint16_t* x, bool planes_ready, uint8_t* xplanes, const uint8_t* pool,
                       const Layout& L, const ExpertSource& src, int32_t* ws_slots, float* ws_w, int D, int F,
                       int k, float limit, const uint16_t* addend, float* routed, uint16_t* out, uint8_t* hid,
                       hipStream_t s, const fp8::DecodeArgs* sh_gu, const fp8::DecodeArgs* sh_dn) {
  if (!planes_ready) {
    hipLaunchKernelGGL(x_planes_kernel, dim3((D / 4 + 255) / 256), dim3(256), 0, s, x, D, xplanes);
    const int rc = check_launch("x_planes_kernel");
    if (rc) return rc;
  }
  const bool sh = sh_gu != nullptr;
  const int NQ = D / 512;
  const int mg = (NQ + GU_WAVES - 1) / GU_WAVES;
  const int n_sh = sh ? sh_gu->N / 8 : 0;
  const dim3 grid_gu(n_sh + k * (F / 16));
#define CACHALOT_GU(MV)                                                                                            \
  if (sh)                                                                                                          \
    hipLaunchKernelGGL((q2mx_gate_up_shared_kernel<MV>), grid_gu, dim3(GU_THREADS), 0, s, xplanes, pool, L, src, D, \
                       F, limit, hid, ws_slots, ws_w, *sh_gu, n_sh);                                               \
  else                                                                                                             \
    hipLaunchKernelGGL((q2mx_gate_up_kernel<MV>), grid_gu, dim3(GU_THREADS), 0, s, xplanes, pool, L, src, D, F,     \
                       limit, hid, ws_slots, ws_w)
  if (mg <= 2) CACHALOT_GU(2);
  else CACHALOT_GU(3);
#undef CACHALOT_GU
  int rc = check_launch("q2mx_gate_up_kernel");
  if (rc) return rc;
  const int NQ2 = ((F + 127) / 128 + 3) / 4;
  const int md = (k * NQ2 + DN_WAVES - 1) / DN_WAVES;
  const fp8::DecodeArgs none{};
#define CACHALOT_DN(MV, SHV)                                                                                     \
  hipLaunchKernelGGL((q2mx_down_kernel<MV, SHV>), dim3(D / 16), dim3(DN_THREADS), 0, s, pool, L, ws_slots, D, F, k, \
                     hid, addend, routed, out, sh ? *sh_dn : none)
  if (md <= 3) {
    if (sh) CACHALOT_DN(3, true);
    else CACHALOT_DN(3, false);
  } else {
    if (sh) CACHALOT_DN(4, true);
    else CACHALOT_DN(4, false);
  }
#undef CACHALOT_DN
  return check_launch("q2mx_down_kernel");
}

// Batched decode over expert-major rows (grouped.hip's permutation): x planes of the
// T tokens and the active experts' records (recs, n_recs: min(E, T k) entries of
// workspace), then gate/up and down over the active experts.
// hid holds rows x GK plane blocks and xplanes T x D / 128.
int launch_q2mx_batched(const uint16_t* x, int T, const uint8_t* pool, const Layout& L, const int32_t* slot_table,
                        const int32_t* offsets, int E, int4* recs, int32_t* n_recs, int max_active,
                        const int32_t* row_token, const int32_t* row_slot, const float* row_w, int D, int F, int k,
                        float limit, uint8_t* hid, uint8_t* xplanes, uint16_t* y, hipStream_t s,
                        const int32_t* ridx, const float* rw) {
  // with routes (T k <= PREP_THREADS) the prep launch permutes them itself into offsets / row_*
  if (ridx != nullptr && T * k > PREP_THREADS) return fail(CACHALOT_EINVAL, "batched decode: %d routes", T * k);
  hipLaunchKernelGGL(batch_prep_kernel, dim3((ridx ? 1 : 2) + T * ((D + 4095) / 4096)), dim3(PREP_THREADS), 0, s, x,
                     T, D, xplanes, const_cast<int32_t*>(offsets), E, slot_table, recs, n_recs, T * k, k,
                     const_cast<int32_t*>(row_token), const_cast<int32_t*>(row_slot), y, ridx, rw,
                     const_cast<float*>(row_w));
  int rc = check_launch("batch_prep_kernel");
  if (rc) return rc;
  BatchArgs a{xplanes, pool, L, recs, n_recs, row_token, row_slot, row_w, D, F, k, limit, hid, y};
  const int NQ = D / 512;
  const int mg = (NQ + GU_WAVES - 1) / GU_WAVES;
  const dim3 grid_gu(F / 16, max_active);
  if (mg <= 2) hipLaunchKernelGGL(q2mx_bgu_kernel<2>, grid_gu, dim3(GU_THREADS), 0, s, a);
  else hipLaunchKernelGGL(q2mx_bgu_kernel<3>, grid_gu, dim3(GU_THREADS), 0, s, a);
  rc = check_launch("q2mx_bgu_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(q2mx_bdn4_kernel, dim3(D / 64, max_active), dim3(GU_THREADS), 0, s, a);
  return check_launch("q2mx_bdn4_kernel");
}

}  // namespace cachalot
