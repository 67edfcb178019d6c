// Decode (one token) over a 2-bit affine g128 bank in ONE persistent launch:
// gate/up GEMV -> SwiGLU -> grid-wide publication of the hidden vectors ->
// down GEMV -> route-order combine.  One 1024-thread workgroup per CU.
//
// Reference semantics: src/cachalot/model/expert_affine.py:65-81 (bf16 g, u,
// h, y_e rounding points), :117-152 (experts summed in route order from zero),
// mx.quantized_matmul's group formula s * sum(x q) + b * sum(x) (as copied at
// minimax/codes_qmv.py:86-100).
//
// Why one launch.  A token-layer reads ~60 MB of codes; at ~6 TB/s that is
// ~10 us, of the order of two kernel launches plus two HBM round trips.  Here
// every workgroup issues all its gate/up code loads at once, the down-proj
// code loads follow as soon as its first gate/up item is consumed (so HBM
// serves gate/up bytes first and streams W2 while the hidden vectors are
// exchanged), and the only grid-wide wait is the hidden-vector barrier.
//
// Work split (G workgroups, 16 waves each):
//   gate/up: the k*F/16 tiles of 16 rows (expert-major) are cut into G
//     contiguous ranges; a workgroup's items are (tile, quad of four 128-code
//     groups), dealt round-robin to its 16 waves.  Each item is one 16x128x4
//     block-scaled MFMA chain per matrix (W1 and W3 share the A operand).
//   publication: wave 15 sums the per-quad partials in a fixed order, applies
//     bf16(g), bf16(u), clamp, h = bf16(silu(g) * u * w_e) and writes each
//     16-row tile of h as one fp8 plane piece (mx_tile.h) with agent-scope
//     stores, then arrives at the grid barrier.
//   down: the D/16 output tiles are cut into G ranges; items are (tile,
//     expert, quad), dealt to waves 0..14 (wave 15 holds no W2 loads, so its
//     store-completion wait before arriving does not wait on them).  After the
//     barrier every workgroup copies the k plane blocks of h into LDS; each
//     expert's row value is rounded to bf16 and the experts are summed in
//     route order (no atomics: deterministic).
#include "decode_common.h"
#include "grid_sync.h"
#include "mfma_tile.h"
#include "mx_tile.h"
#include "router_launch.h"

namespace cachalot {
namespace {

using namespace decode;
using mx::f32x4_t;
using mx::i32x8_t;
using mx::PB_BYTES;
using mx::PB_SCALE;
using mx::PB_SUM;
using mx::ARole;
using mx::Chain;
using mx::a_role;
using mx::chain_init;
using mx::chain_load;
using mx::dot4;
using mx::piece_sums;
using mx::lds16;
using mx::bf16_lo;

constexpr int THREADS = 1024;
constexpr int WAVES = THREADS / 64;
constexpr int PUB = WAVES - 1;           // publishing wave: h pieces, grid barrier; no down items
constexpr int DN_WAVES = WAVES - 1;      // waves holding down items (their W2 loads stay in flight
                                         // while the publishing wave waits for its stores)
constexpr int MAX_GT = 40;               // D <= 5120
constexpr int MAX_NQ = MAX_GT / 4;
constexpr int MAX_GK = 24;               // F <= 3072
constexpr int MAX_NQ2 = MAX_GK / 4;
constexpr int MAX_T = 6;                 // gate/up tiles per workgroup
constexpr int MAX_TD = 2;                // down tiles per workgroup
constexpr int MAX_GU_ITEMS = WAVES * 3;
constexpr int MAX_DN_ITEMS = DN_WAVES * 4;
constexpr int MAX_E = 1024;
constexpr int PLANE_LDS = KMAX * MAX_GK * PB_BYTES;   // >= MAX_GT * PB_BYTES

// Phase timestamps for tuning: compiled only with -DCACHALOT_TRACE_PHASES, when the
// launcher takes the buffer from the CACHALOT_TRACE environment variable
// (16 x u64 per workgroup, s_memrealtime ticks at 100 MHz).
#ifdef CACHALOT_TRACE_PHASES
#define PHASE(i)                                                                                    \
  do {                                                                                              \
    if (p.trace && (tid & 63) == 0 && (tid >> 6) == PUB)                                            \
      p.trace[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                            \
  } while (0)
#else
#define PHASE(i) \
  do {           \
  } while (0)
#endif

struct FusedQ2 {
  const uint16_t* x;
  const uint8_t* pool;
  Layout L;
  const int32_t* slot_table;
  const int32_t* idx;       // null: experts from ws_slots / ws_w (router tail)
  const float* w;
  const int32_t* ws_slots;
  const float* ws_w;
  int E, D, F, k;
  float limit;
  const uint16_t* addend;
  float* routed;
  uint16_t* out;
  uint8_t* sync;            // gsync block
  uint8_t* hid;             // k * GK plane blocks
  unsigned long long* trace;
};

struct Lds {
  uint8_t planes[PLANE_LDS];                          // x planes during gate/up, then h planes
  uint8_t zero[64];                                   // A data of pieces past the end of a vector
  // per wave, per gate/up item: [s1, b1, s3, b3][16 rows] 16-byte chunks holding the
  // item's four groups
  uint8_t scl[WAVES][3][1024];
  float red_gu[MAX_T][MAX_NQ][2][16];
  float red_dn[MAX_TD][KMAX][MAX_NQ2][16];
  int32_t slots[MAX_E];
  uint32_t stage[MAX_T][10];   // per tile: hi plane (4 words), lo plane (4), scales, sum
  int32_t eslot[KMAX];
  float ew[KMAX];
  // per-workgroup item tables (no integer division in the item loops)
  uint8_t gu_tl[MAX_GU_ITEMS], gu_q[MAX_GU_ITEMS];
  uint8_t dn_tdl[MAX_DN_ITEMS], dn_e[MAX_DN_ITEMS], dn_q2[MAX_DN_ITEMS];
  int16_t t_e[MAX_T], t_p[MAX_T];                     // tile -> expert, 16-row piece within the expert
};

template <int MAXGU, int MAXDN, int XP>
__global__ void __launch_bounds__(THREADS) q2_decode_fused_kernel(FusedQ2 p) {
  __shared__ __align__(16) Lds s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: role branches are uniform
  const int j = lane & 15, kg = lane >> 4;
  const int G = gridDim.x, b = blockIdx.x;
  const int D = p.D, F = p.F, k = p.k;
  const int GT = D / 128, NQ = GT / 4;
  const int GK = (F + 127) / 128, NQ2 = (GK + 3) / 4;
  const int FT = F / 16;                       // 16-row tiles (= plane pieces) per expert
  const uint32_t gen = gsync::next_generation(p.sync);
  PHASE(0);

  // gate/up: ceil(TT / G) tiles per workgroup on the first ceil(TT / that) workgroups,
  // so every workgroup with gate/up work streams the same number of bytes (the last
  // one excepted); the rest only take down work
  const int TT = k * FT;
  const int tpw = (TT + G - 1) / G;
  const int t0 = min(b * tpw, TT), t1 = min(t0 + tpw, TT);
  const int nt = t1 - t0;
  const int n_gu = nt * NQ;
  const int64_t TD = D / 16;
  const int d0 = (int)(TD * b / G), d1 = (int)(TD * (b + 1) / G);
  const int ntd = d1 - d0;
  const int n_dn = ntd * k * NQ2;

  // ---- 0. x (registers), the slot table, the item tables
  uint2 xr[XP];   // 4 bf16 of x per lane and pass
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int t4 = tid + THREADS * i;
    xr[i] = 4 * t4 < D ? reinterpret_cast<const uint2*>(p.x)[t4] : make_uint2(0, 0);
  }
  if (p.idx && tid < p.E) s.slots[tid] = p.slot_table[tid];
  // every entry is written (items past a workgroup's count point at valid tiles and
  // experts): a workgroup may have no gate/up or no down items at all
  if (tid < MAX_GU_ITEMS) {
    const bool v = tid < n_gu;
    s.gu_tl[tid] = (uint8_t)(v ? tid / NQ : 0);
    s.gu_q[tid] = (uint8_t)(v ? tid % NQ : 0);
  }
  if (tid < MAX_DN_ITEMS) {
    const bool v = tid < n_dn;
    s.dn_tdl[tid] = (uint8_t)(v ? tid / (k * NQ2) : 0);
    s.dn_e[tid] = (uint8_t)(v ? (tid / NQ2) % k : 0);
    s.dn_q2[tid] = (uint8_t)(v ? tid % NQ2 : 0);
  }
  if (tid < MAX_T) {
    const bool v = tid < nt;
    s.t_e[tid] = (int16_t)(v ? (t0 + tid) / FT : 0);
    s.t_p[tid] = (int16_t)(v ? (t0 + tid) % FT : 0);
  }
  if (tid < 16) reinterpret_cast<uint32_t*>(s.zero)[tid] = 0u;
  lds_sync();
  if (tid < k) {
    int slot;
    float we;
    if (p.idx) {
      const int ex = p.idx[tid];
      slot = (ex >= 0 && ex < p.E) ? s.slots[ex] : -1;
      we = p.w[tid];
    } else {
      slot = p.ws_slots[tid];
      we = p.ws_w[tid];
    }
    s.eslot[tid] = slot;
    s.ew[tid] = we;
  }
  lds_sync();
  PHASE(1);


  // ---- 1. x as fp8 planes in LDS (a quad of lanes per 16-element piece), before any
  //         code load is issued: a CU cannot hold them all in flight, so waves stall at
  //         issue until earlier loads land, and nothing queued behind them may be needed.
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int t4 = tid + THREADS * i;
    if (4 * t4 < D) mx::encode_x_quad(s.planes, t4, xr[i]);   // uniform per quad
  }
  lds_sync();
  PHASE(2);
  // ---- 2. gate/up loads.  Per item: one direct-to-LDS copy of the scale / bias chunks
  //         (lane = tensor x row), then the codes.  The copy is issued first, so the
  //         wait for an item's codes (loads complete in issue order) covers it too.
  uint4 c1[MAXGU][2], c3[MAXGU][2];
  const uint4 sc_off = make_uint4((uint32_t)p.L.off[1], (uint32_t)p.L.off[2], (uint32_t)p.L.off[7],
                                  (uint32_t)p.L.off[8]);   // records are < 4 GiB
  int gsb[MAXGU];   // byte of the item's first group inside its scale chunks
  auto gu_load = [&](int m) {
    const int it = min(wave + WAVES * m, max(n_gu - 1, 0));
    const int tl = s.gu_tl[it], q = s.gu_q[it];
    const int slot = max(s.eslot[min((int)s.t_e[tl], k - 1)], 0);
    const int row0 = s.t_p[tl] * 16;
    const uint8_t* base = p.pool + (int64_t)slot * p.L.record_bytes;
    {
      const int t = lane >> 4, r = lane & 15;
      const int toff = (int)(t == 0 ? sc_off.x : t == 1 ? sc_off.y : t == 2 ? sc_off.z : sc_off.w);
      const int o = ((row0 + r) * GT + 4 * q) * 2;
      tile::lds_load16_untracked(base + (uint32_t)(toff + (o & ~15)), s.scl[wave][m]);
      gsb[m] = (8 * q) & 15;
    }
    const int64_t off = (int64_t)(row0 + j) * (D / 4) + (4 * q + kg) * 32;
    const uint4* r1 = reinterpret_cast<const uint4*>(base + p.L.off[0] + off);
    const uint4* r3 = reinterpret_cast<const uint4*>(base + p.L.off[6] + off);
    c1[m][0] = r1[0];
    c1[m][1] = r1[1];
    c3[m][0] = r3[0];
    c3[m][1] = r3[1];
  };
  if (n_gu > 0) {   // uniform over the workgroup
#pragma unroll
    for (int m = 0; m < MAXGU; ++m) gu_load(m);
  }


  const ARole ro = a_role(lane);
  Chain CH;   // persistent A operands of the current chain
  chain_init(CH);

  // ---- 3. gate/up items
  auto gu_item = [&](int m) {
    const int it = wave + WAVES * m;
    if (it >= n_gu) return;
    const int tl = s.gu_tl[it], q = s.gu_q[it];
    if (s.eslot[s.t_e[tl]] < 0) return;   // the publication writes zero rows
    // the item's last code load has landed, hence (loads complete in issue order) its
    // earlier scale copy too; no LDS read of the scales may move above this point
    asm volatile("" ::"v"(c3[m][1].w) : "memory");
    const uint8_t* blkA = s.planes + (4 * q + ro.kgR) * PB_BYTES;
    f32x4_t a1 = mx::zero_acc<true>(), a3 = mx::zero_acc<true>();
    chain_load(CH, blkA, ro);
    const uint4& u1a = c1[m][0];
    const uint4& u1b = c1[m][1];
    const uint4& u3a = c3[m][0];
    const uint4& u3b = c3[m][1];
    a1 = mx::mfma_fp8_fp4<0, true>(CH.a[0], mx::q2_spread(u1a.x, u1a.y), a1, CH.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<0, true>(CH.a[0], mx::q2_spread(u3a.x, u3a.y), a3, CH.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<1, true>(CH.a[1], mx::q2_spread(u1a.z, u1a.w), a1, CH.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<1, true>(CH.a[1], mx::q2_spread(u3a.z, u3a.w), a3, CH.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<2, true>(CH.a[2], mx::q2_spread(u1b.x, u1b.y), a1, CH.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<2, true>(CH.a[2], mx::q2_spread(u3b.x, u3b.y), a3, CH.sa, mx::E8M0_TWO);
    a1 = mx::mfma_fp8_fp4<3, true>(CH.a[3], mx::q2_spread(u1b.z, u1b.w), a1, CH.sa, mx::E8M0_TWO);
    a3 = mx::mfma_fp8_fp4<3, true>(CH.a[3], mx::q2_spread(u3b.z, u3b.w), a3, CH.sa, mx::E8M0_TWO);
    const float sx = piece_sums(s.planes + (4 * q + kg) * PB_BYTES, mx::PIECES);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(s.scl[wave][m]) + (j * 16 + gsb[m] + 2 * kg) / 2;
    const float v1 = bf16_to_f32(sc[0]) * dot4(a1) + bf16_to_f32(sc[128]) * sx;
    const float v3 = bf16_to_f32(sc[256]) * dot4(a3) + bf16_to_f32(sc[384]) * sx;
    const float r1 = tile::sum_lane_groups(v1);
    const float r3 = tile::sum_lane_groups(v3);
    if (lane < 16) {
      s.red_gu[tl][q][0][lane] = r1;
      s.red_gu[tl][q][1][lane] = r3;
    }
  };

  // W2 codes of this wave's down items, spread into B operands ahead of the barrier
  uint4 c2[MAXDN][2] = {};   // (the publishing wave loads none)
  uint32_t dsc[MAXDN][2];
  auto dn_load = [&]() {
#pragma unroll
    for (int m = 0; m < MAXDN; ++m) {
      const int it = min(wave + DN_WAVES * m, max(n_dn - 1, 0));
      const int tdl = s.dn_tdl[it], e = min((int)s.dn_e[it], k - 1), q2 = s.dn_q2[it];
      const int slot = max(s.eslot[e], 0);
      const int g2 = min(4 * q2 + kg, GK - 1);
      const int n = min(d0 + tdl, (int)TD - 1) * 16 + j;
      const uint8_t* base = p.pool + (int64_t)slot * p.L.record_bytes;
      const uint4* r2 = reinterpret_cast<const uint4*>(base + p.L.off[3] + (int64_t)n * (GK * 32) + g2 * 32);
      c2[m][0] = r2[0];
      c2[m][1] = r2[1];
      const int64_t si = ((int64_t)n * GK + g2) * 2;
      dsc[m][0] = *reinterpret_cast<const uint16_t*>(base + p.L.off[4] + si);
      dsc[m][1] = *reinterpret_cast<const uint16_t*>(base + p.L.off[5] + si);
    }
  };

  // down-item descriptors (wave-uniform), decoded before the barrier
  bool dn_on[MAXDN];
  int dn_tv[MAXDN], dn_ev[MAXDN], dn_qv[MAXDN];
#pragma unroll
  for (int m = 0; m < MAXDN; ++m) {
    const int it = wave + DN_WAVES * m;
    const int itc = min(it, max(n_dn - 1, 0));
    dn_tv[m] = s.dn_tdl[itc];
    dn_ev[m] = s.dn_e[itc];
    dn_qv[m] = s.dn_q2[itc];
    dn_on[m] = wave != PUB && it < n_dn && s.eslot[dn_ev[m]] >= 0;
  }

  // the W2 loads follow the wave's last gate/up item: HBM serves gate/up first and
  // streams W2 while the hidden vectors are published and exchanged
#pragma unroll
  for (int m = 0; m < MAXGU; ++m) gu_item(m);
  if (wave != PUB && n_dn > 0) dn_load();
  PHASE(3);
  lds_sync();
  PHASE(4);

  // ---- 4. publication of h and the grid barrier.  Wave t < nt finishes tile t (16
  //         rows) into LDS staging; the publishing wave then writes every tile with
  //         one store instruction (lane = tile x word) and arrives.
  uint8_t* bar = p.sync;
  if (wave < nt && lane < 16) {
    const int tl = wave, r = lane;
    const int e = s.t_e[tl];
    float hv = 0.0f;
    if (s.eslot[e] >= 0) {
      float g = 0.0f, u = 0.0f;
      for (int q = 0; q < NQ; ++q) {
        g = g + s.red_gu[tl][q][0][r];
        u = u + s.red_gu[tl][q][1][r];
      }
      g = round_bf16(g);
      u = round_bf16(u);
      if (p.limit > 0.0f) {
        u = fminf(fmaxf(u, -p.limit), p.limit);
        g = fminf(g, p.limit);
      }
      hv = round_bf16((silu_f32(g) * u) * s.ew[e]);
    }
    const mx::PieceCode pc = mx::encode_piece(hv);
    uint8_t* st = reinterpret_cast<uint8_t*>(s.stage[tl]);
    st[mx::piece_pos(r)] = (uint8_t)pc.hi;
    st[16 + mx::piece_pos(r)] = (uint8_t)pc.lo;
    if (r == 0) {
      s.stage[tl][8] = pc.scales;
      s.stage[tl][9] = __float_as_uint(pc.sum);
    }
  }
  lds_sync();
  if (wave == PUB) {
    // per tile: 11 stores (hi plane 4 words, lo plane 4 words, 2 scale bytes, sum),
    // plus, for the last tile of an expert, the same for every piece of its group past
    // F, as zeros (so consumers read whole steps unmasked)
    for (int tl = 0; tl < nt; ++tl) {
      const int e = s.t_e[tl], P = s.t_p[tl];
      const int extra = (P == FT - 1) ? 7 - (P & 7) : 0;
      uint8_t* blk = p.hid + ((int64_t)e * GK + (P >> 3)) * PB_BYTES;
      for (int i = lane; i < 11 * (1 + extra); i += 64) {
        const int pc = i / 11, w = i - 11 * pc;
        const int pp = (P & 7) + pc;
        const bool zero = pc > 0;
        if (w < 8) {
          const uint32_t v = zero ? 0u : s.stage[tl][w];
          gsync::store_agent(reinterpret_cast<uint32_t*>(blk + mx::pb_data(pp, w >> 2) + 4 * (w & 3)), v);
        } else if (w < 10) {
          const uint8_t v = zero ? (uint8_t)127 : (uint8_t)(s.stage[tl][8] >> (8 * (w - 8)));
          __hip_atomic_store(blk + mx::pb_scale(pp, w - 8), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          gsync::store_agent(reinterpret_cast<uint32_t*>(blk + PB_SUM + 4 * pp), zero ? 0u : s.stage[tl][9]);
        }
      }
    }
    tile::wait_vmem();
    PHASE(5);
    if (lane == 0) gsync::arrive(bar);
    PHASE(6);
    gsync::wait(bar, p.sync, gen, lane);
    PHASE(7);
  }

  // W2 codes -> B operands while the barrier completes
  i32x8_t B2[MAXDN][4];
#pragma unroll
  for (int m = 0; m < MAXDN; ++m) {
    B2[m][0] = mx::q2_spread(c2[m][0].x, c2[m][0].y);
    B2[m][1] = mx::q2_spread(c2[m][0].z, c2[m][0].w);
    B2[m][2] = mx::q2_spread(c2[m][1].x, c2[m][1].y);
    B2[m][3] = mx::q2_spread(c2[m][1].z, c2[m][1].w);
  }
  lds_sync();

  // ---- 5. h planes into LDS (agent-coherent copy), then the down items
  tile::dma_to_lds<1>(p.hid, s.planes, k * GK * PB_BYTES, wave, WAVES, lane);
  tile::wait_vmem();
  lds_sync();
  PHASE(8);

#pragma unroll
  for (int m = 0; m < MAXDN; ++m) {
    if (!dn_on[m]) continue;
    const int e = dn_ev[m], q2 = dn_qv[m];
    const uint8_t* blkA = s.planes + (e * GK + min(4 * q2 + ro.kgR, GK - 1)) * PB_BYTES;
    const int g2 = 4 * q2 + kg;
    const float sh = g2 < GK ? piece_sums(s.planes + (e * GK + g2) * PB_BYTES, min(8, FT - 8 * g2)) : 0.0f;
    f32x4_t acc = mx::zero_acc<true>();
    chain_load(CH, blkA, ro);
    acc = mx::mfma_fp8_fp4<0, true>(CH.a[0], B2[m][0], acc, CH.sa, mx::E8M0_TWO);
    acc = mx::mfma_fp8_fp4<1, true>(CH.a[1], B2[m][1], acc, CH.sa, mx::E8M0_TWO);
    acc = mx::mfma_fp8_fp4<2, true>(CH.a[2], B2[m][2], acc, CH.sa, mx::E8M0_TWO);
    acc = mx::mfma_fp8_fp4<3, true>(CH.a[3], B2[m][3], acc, CH.sa, mx::E8M0_TWO);
    float v = g2 < GK ? bf16_lo(dsc[m][0]) * dot4(acc) + bf16_lo(dsc[m][1]) * sh : 0.0f;
    v = tile::sum_lane_groups(v);
    if (lane < 16) s.red_dn[dn_tv[m]][e][q2][lane] = v;
  }
  lds_sync();
  PHASE(9);

  // ---- 6. route-order combine of this workgroup's output rows
  if (tid < ntd * 16) {
    const int tdl = tid >> 4, r = tid & 15;
    const int n = (d0 + tdl) * 16 + r;
    float total = 0.0f;
    for (int e = 0; e < k; ++e) {
      float y = 0.0f;
      if (s.eslot[e] >= 0)
        for (int q2 = 0; q2 < NQ2; ++q2) y = y + s.red_dn[tdl][e][q2][r];
      total = total + round_bf16(y);
    }
    if (p.routed) p.routed[n] = total;
    if (p.out) p.out[n] = f32_to_bf16(p.addend ? total + bf16_to_f32(p.addend[n]) : total);
  }
  if (b == 0 && tid == 0) gsync::finish(p.sync, gen);
  PHASE(10);
}

struct DeviceInfo {
  int cus = 0;
  bool fits = false;
};

DeviceInfo device_info() {
  static thread_local int cached_dev = -1;
  static thread_local DeviceInfo cached;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return DeviceInfo{};
  if (dev == cached_dev) return cached;
  DeviceInfo d;
  if (hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) d.cus = 0;
  int per = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(q2_decode_fused_kernel<3, 4, 8>),
                                                   THREADS, 0) == hipSuccess)
    d.fits = per >= 1;
  cached = d;
  cached_dev = dev;
  return d;
}

}  // namespace

static_assert(gsync::BYTES <= WS_SYNC_BYTES, "grid-barrier block must fit its workspace slot");

// Bytes after the two-kernel layout: the k hidden-vector plane blocks.
size_t q2_fused_region_bytes(int F, int k) {
  const int GK = (F + 127) / 128;
  return align256((size_t)k * GK * PB_BYTES);
}

// The fused path's shape envelope; returns the grid size (0: use the two-kernel path).
int q2_fused_grid(int D, int F, int k) {
  // opt-in while the two-kernel path is faster (CACHALOT_DECODE_FUSED=1)
  const char* env = getenv("CACHALOT_DECODE_FUSED");
  if (!env || env[0] != '1') return 0;
  if (D % 1024 != 0 || D > 128 * MAX_GT || F % 64 != 0 || F > 128 * MAX_GK || k < 1 || k > KMAX) return 0;
  const DeviceInfo di = device_info();
  if (di.cus <= 0 || !di.fits) return 0;
  const int G = di.cus;
  const int64_t FT = F / 16, TT = (int64_t)k * FT, TD = D / 16;
  const int max_t = (int)((TT + G - 1) / G);          // tiles per gate/up workgroup
  const int max_td = (int)((TD + G - 1) / G);
  if (max_t > MAX_T || max_td > MAX_TD) return 0;
  const int NQ = D / 512, NQ2 = ((F + 127) / 128 + 3) / 4;
  if ((max_t * NQ + WAVES - 1) / WAVES > 3) return 0;
  if ((max_td * k * NQ2 + DN_WAVES - 1) / DN_WAVES > 4) return 0;
  return G;
}

int launch_q2_decode_fused(int G, const uint16_t* x, const uint8_t* pool, const Layout& L, const ExpertSource& src,
                           const int32_t* ws_slots, const float* ws_w, int D, int F, int k, float limit,
                           const uint16_t* addend, float* routed, uint16_t* out, uint8_t* sync, uint8_t* hid,
                           hipStream_t s) {
  FusedQ2 p;
  p.x = x;
  p.pool = pool;
  p.L = L;
  p.slot_table = src.slot_table;
  p.idx = src.idx;
  p.w = src.w;
  p.ws_slots = ws_slots;
  p.ws_w = ws_w;
  p.E = src.E;
  p.D = D;
  p.F = F;
  p.k = k;
  p.limit = limit;
  p.addend = addend;
  p.routed = routed;
  p.out = out;
  p.sync = sync;
  p.hid = hid;
  p.trace = nullptr;
#ifdef CACHALOT_TRACE_PHASES
  if (const char* t = getenv("CACHALOT_TRACE")) p.trace = reinterpret_cast<unsigned long long*>(strtoull(t, nullptr, 0));
#endif
  const int xp = (D + 4095) / 4096;
  const int64_t TT = (int64_t)k * (F / 16), TD = D / 16;
  const int max_t = (int)((TT + G - 1) / G), max_td = (int)((TD + G - 1) / G);
  const int mgu = (max_t * (D / 512) + WAVES - 1) / WAVES;
  const int mdn = (max_td * k * (((F + 127) / 128 + 3) / 4) + DN_WAVES - 1) / DN_WAVES;
#define CACHALOT_FQ2(MG, MD, XPV) \
  hipLaunchKernelGGL((q2_decode_fused_kernel<MG, MD, XPV>), dim3(G), dim3(THREADS), 0, s, p)
  if (xp <= 1) {
    if (mgu <= 2 && mdn <= 3) CACHALOT_FQ2(2, 3, 1);
    else if (mdn <= 3) CACHALOT_FQ2(3, 3, 1);
    else CACHALOT_FQ2(3, 4, 1);
  } else {
    if (mdn <= 3) CACHALOT_FQ2(3, 3, 2);
    else CACHALOT_FQ2(3, 4, 2);
  }
#undef CACHALOT_FQ2
  return check_launch("q2_decode_fused_kernel");
}

}  // namespace cachalot
