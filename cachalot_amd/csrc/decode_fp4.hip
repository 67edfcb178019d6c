// Decode (one token) over an FP4 E2M1 / E8M0-block-32 expert bank, on the matrix cores.
//
// Reference: src/cachalot/model/moe_fused_metal.py:189-233 (fused_gate_up +
// fused_down): x read as fp32, gate/up accumulated in fp32,
// h = silu(min(g, L)) * clip(u, -L, L) * w_e in fp32 (:127-135), out = sum_e
// W2_e h_e in fp32 with experts in route order (:160-178).  No bf16 rounding
// point anywhere on this path.
//
// A "piece" is 32 codes of a row: 16 bytes of nibbles and one E8M0 scale.  The
// converter turns a nibble word into 8 exact bf16 values (E2M1 x 2^e), which
// meet bf16 activations in v_mfma_f32_16x16x32_bf16 (exact products, fp32 sums).
//
//   fp4_gate_up_kernel  one workgroup = one expert x one 16-row tile of W1 and
//                       W3; four waves split K into quarters; lane group kg of
//                       block b takes piece 4b + kg of the wave's quarter (one
//                       load instruction covers whole 64-byte runs of a row).
//                       Every A row carries x, so D[i][j] is the dot product of
//                       weight row j for every i.  Epilogue in fp32:
//                       h = silu(min(g, L)) * clip(u, +-L) * w_e.
//   fp4_down_kernel     one workgroup = one 16-row tile of W2 for all k experts,
//                       2k waves (expert, K half).  The fp32 hidden vectors are
//                       staged in LDS as bf16 hi + lo parts (A rows 0 and 1:
//                       h = hi + lo to 16 significant bits); expert row values
//                       are summed in fp32 in route order.
#include "decode_common.h"
#include "fp8_common.h"
#include "mfma_tile.h"
#include "router_launch.h"

namespace cachalot {
namespace {

using namespace decode;
using namespace tile;

constexpr int GU_WAVES = 4;
constexpr int DN_HALVES = 2;
constexpr int PIECE = 32;                        // codes per piece (one E8M0 scale)
constexpr int MAX_D = 8192;
constexpr int MAX_KF = 24576;                    // k * F staged by the down kernel
constexpr int ZERO_BYTES = 64;                   // 4 steps x 16 bytes
constexpr int GU_ZERO = MAX_D * 2;

// Copy `bytes` (a multiple of 16) into LDS with untracked direct-to-LDS loads, 1 KiB
// chunks c = part, part + parts, ... (tile::lds_load16_untracked); the caller waits.
__device__ __forceinline__ void copy_untracked(const void* src, uint8_t* dst, int bytes, int part, int parts,
                                               int lane) {
  for (int c = __builtin_amdgcn_readfirstlane(part) * 1024; c < bytes; c += parts * 1024)
    if (c + 16 * lane < bytes)
      lds_load16_untracked(reinterpret_cast<const uint8_t*>(src) + c + 16 * lane, dst + c);
}

// s_waitcnt with vmcnt(n), expcnt and lgkmcnt unconstrained (gfx9 encoding, n < 64).
#define VMCNT(n) (0x0F70 | ((n) & 15) | (((n) >> 4) << 14))

template <int NB>
__device__ __forceinline__ void lane_pieces(int first, int PW, int pieces, int kg, int (&pi)[NB], bool (&pv)[NB]) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int within = 4 * b + kg;
    const int P = first + within;
    pv[b] = within < PW && P < pieces;
    pi[b] = min(P, pieces - 1);
  }
}

// grid.x = k * F / 16 + n_sh: the routed tiles, then n_sh tiles of the FP8 shared
// expert's gate/up (fp8::shared_gu_tile, h_sh to sh.out; they need no routing, so they
// go last, into the slots the first routed workgroups leave).
// NB = ceil(ceil(D/32 / 4) / 4); XI = ceil(D / 4096).
template <int NB, int XI, bool SH>
__global__ void __launch_bounds__(64 * GU_WAVES) fp4_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L, ExpertSource src, int D, int F,
    float limit, uint16_t* __restrict__ hidden, int32_t* __restrict__ ws_slots,
    float* __restrict__ ws_w, fp8::DecodeArgs sh, int n_sh) {
  __shared__ __align__(16) uint8_t xl[GU_ZERO + ZERO_BYTES];
  __shared__ __align__(16) uint8_t sc[2 * 16 * (MAX_D / PIECE)];   // s1, s3 of the tile's rows
  __shared__ float red[GU_WAVES][2][16];
  static_assert(GU_ZERO + ZERO_BYTES >= fp8::dec_tile_lds(1, fp8::SH_MAX_K), "shared tile LDS");
  if constexpr (SH) {
    if ((int)blockIdx.x >= (int)gridDim.x - n_sh) {
      fp8::shared_gu_tile<64 * GU_WAVES>(sh, blockIdx.x - (gridDim.x - n_sh), xl);
      return;
    }
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int PT = D / PIECE;
  const int tiles = F / 16;
  const int e = blockIdx.x / tiles;
  const int tile = blockIdx.x - e * tiles;
  const int row0 = tile * 16;
  __shared__ int top_i[GU_WAVES][KMAX];
  __shared__ float top_v[GU_WAVES][KMAX], top_w[GU_WAVES][KMAX];
  __shared__ int top_s[GU_WAVES][KMAX];
  const int slot = route_slot(src, ws_slots, e, top_i[wave], top_v[wave], top_s[wave]);
  // the slot for the down kernel is stored at the end (a store's data registers stay
  // busy until it completes, and the compiler would wait for it before the loads)
  const bool store_slot = src.scores && tile == 0 && threadIdx.x == 0;
  uint16_t* hout = hidden + (size_t)e * F * 2;   // per expert: hi [F], lo [F] (bf16)
  if (slot < 0) {
    if (store_slot) ws_slots[e] = slot;
    if (threadIdx.x < 16) {
      hout[row0 + threadIdx.x] = hout[F + row0 + threadIdx.x] = 0;
      route_finish(src, ws_w, e, tile, top_v[0], top_w[0], top_i[0], blockIdx.x == 0);
    }
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const int j = lane & 15, kg = lane >> 4;
  const int row = row0 + j;
  const int PW = (PT + GU_WAVES - 1) / GU_WAVES;
  int pi[NB];
  bool pv[NB];
  lane_pieces<NB>(wave * PW, PW, PT, kg, pi, pv);

  // the tile's scales (two runs of 16 rows x PT bytes) and the activations into LDS
  // first, then the codes; the barrier waits for the copies only, and each block of
  // codes is consumed as it lands
  copy_untracked(base + L.off[1] + (int64_t)row0 * PT, sc, 16 * PT, wave, GU_WAVES, lane);
  copy_untracked(base + L.off[7] + (int64_t)row0 * PT, sc + 16 * PT, 16 * PT, (wave + 2) & 3, GU_WAVES, lane);
  copy_untracked(x, xl, D * 2, wave, GU_WAVES, lane);
  uint4 wg[NB], wu[NB];
  {
    const uint4* r1 = reinterpret_cast<const uint4*>(base + L.off[0]) + (size_t)row * PT;
    const uint4* r3 = reinterpret_cast<const uint4*>(base + L.off[6]) + (size_t)row * PT;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      wg[b] = r1[pi[b]];
      wu[b] = r3[pi[b]];
    }
  }
  if (threadIdx.x < ZERO_BYTES / 16) reinterpret_cast<uint4*>(xl + GU_ZERO)[threadIdx.x] = make_uint4(0, 0, 0, 0);
  __builtin_amdgcn_s_waitcnt(VMCNT(2 * NB));
  lds_sync();

  f32x4_t cg = {0.0f, 0.0f, 0.0f, 0.0f}, cu = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint32_t aoff = pv[b] ? (uint32_t)pi[b] * (PIECE * 2) : (uint32_t)GU_ZERO;
    const float sg = e8m0_to_f32(sc[j * PT + pi[b]]);
    const float su = e8m0_to_f32(sc[(16 + j) * PT + pi[b]]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8_t a = lds_a(xl, aoff + 16 * s);
      cg = mfma(a, fp4_codes_to_b(word_of(wg[b], s), sg), cg);
      cu = mfma(a, fp4_codes_to_b(word_of(wu[b], s), su), cu);
    }
  }
  if (lane < 16) {
    red[wave][0][lane] = cg[0];
    red[wave][1][lane] = cu[0];
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    if (store_slot) ws_slots[e] = slot;
    const float wexp = route_finish(src, ws_w, e, tile, top_v[0], top_w[0], top_i[0], blockIdx.x == 0);
    const int t = threadIdx.x;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int w = 0; w < GU_WAVES; ++w) {
      g = g + red[w][0][t];
      u = u + red[w][1][t];
    }
    if (limit > 0.0f) {
      u = fminf(fmaxf(u, -limit), limit);
      g = fminf(g, limit);
    }
    const float h = (silu_f32(g) * u) * wexp;
    const uint16_t hi = f32_to_bf16(h);
    hout[row0 + t] = hi;                                         // bf16 hi part
    hout[F + row0 + t] = f32_to_bf16(h - bf16_to_f32(hi));      // bf16 lo part
  }
}

// grid.x = D / 16; block = 64 * k * DN_HALVES.  NB = ceil(ceil(F/32 / 2) / 4).
// SH: the workgroup also runs the FP8 shared expert's down tile of the same 16 rows
// (w2 over act_quant(h_sh), sh.a = h_sh; its 16 w2 rows, h_sh and the scale row in LDS,
// the 2k waves running the 16 virtual waves), whose bf16 y is the addend.  SH holds
// k F <= SH_KF hidden values and a shared F <= SH_F in LDS.
constexpr int SH_KF = 6 * 2880;
constexpr int SH_F = 3072;
template <bool SH>
struct DnShape {
  static constexpr int KF = SH ? SH_KF : MAX_KF;
  static constexpr int THREADS = SH ? 64 * 6 * DN_HALVES : 64 * KMAX * DN_HALVES;
};
template <int NB, bool SH>
__global__ void __launch_bounds__(DnShape<SH>::THREADS) fp4_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, ExpertSource src, const int32_t* __restrict__ ws_slots, int D, int F,
    int k, const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ addend, float* __restrict__ routed,
    uint16_t* __restrict__ out, fp8::DecodeArgs sh) {
  constexpr int KF = DnShape<SH>::KF;
  __shared__ __align__(16) uint8_t hl[KF * 4 + ZERO_BYTES];     // per expert: hi [F] bf16, lo [F] bf16
  __shared__ __align__(16) uint8_t sc[KF / 2];                  // per expert: s2 of the tile's rows
  __shared__ float vals[KMAX][DN_HALVES][16];
  constexpr int SH_TILE = fp8::dec_tile_lds(1, SH_F);
  __shared__ __align__(16) uint8_t sh_lds[SH ? SH_TILE + 18 * SH_F + SH_F / 32 : 16];
  uint8_t* sh_w = sh_lds + SH_TILE;   // the 16 w2 rows (16 K bytes)
  uint8_t* sh_h = sh_w + 16 * SH_F;   // h_sh as copied (bf16)
  uint8_t* sh_sc = sh_h + 2 * SH_F;   // the tile's scale row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int PK = F / PIECE;
  const int e = wave / DN_HALVES;
  const int half = wave - e * DN_HALVES;
  const int row0 = blockIdx.x * 16;
  const int j = lane & 15, kg = lane >> 4;
  const int DNZ = KF * 4;   // the zero bytes after the staged hidden values
  // (shared expert: its scale-row byte first, into LDS at the barrier)
  uint32_t sh_sb = 0;
  if constexpr (SH) sh_sb = sh.ws[0][(size_t)(row0 / 32) * (sh.K / 32) + min((int)threadIdx.x, sh.K / 32 - 1)];
  const int slot = expert_slot(src, ws_slots, e);
  const int PW = (PK + DN_HALVES - 1) / DN_HALVES;
  int pi[NB];
  bool pv[NB];
  lane_pieces<NB>(half * PW, PW, PK, kg, pi, pv);

  // hidden hi / lo parts and, per expert, the tile's scales (16 rows x PK bytes) into
  // LDS first, then the codes (unconditional: a missing expert reads slot 0's bytes and
  // discards them); the barrier waits for the copies only
  // (wave r < k copies expert r's scales: 2k waves >= k; its slot is read with the wave's own)
  const int ps = __builtin_amdgcn_readfirstlane(max(expert_slot(src, ws_slots, min(wave, k - 1)), 0));
  // (both slots are in scalar registers before any copy is issued: a wait for them
  // would otherwise wait for the copies too)
  const int slot_s = __builtin_amdgcn_readfirstlane(slot);
  copy_untracked(hidden, hl, k * F * 4, wave, nwaves, lane);
  if constexpr (SH) copy_untracked(sh.a, sh_h, 2 * sh.K, wave, nwaves, lane);
  if (wave < k)
    copy_untracked(pool + (int64_t)ps * L.record_bytes + L.off[4] + (int64_t)row0 * PK, sc + wave * 16 * PK, 16 * PK,
                   0, 1, lane);
  uint4 wd[NB];
  {
    const uint4* r2 = reinterpret_cast<const uint4*>(pool + (int64_t)max(slot_s, 0) * L.record_bytes + L.off[3]) +
                      (size_t)(row0 + j) * PK;
#pragma unroll
    for (int b = 0; b < NB; ++b) wd[b] = r2[pi[b]];
  }
  if (threadIdx.x < ZERO_BYTES / 16) reinterpret_cast<uint4*>(hl + DNZ)[threadIdx.x] = make_uint4(0, 0, 0, 0);
  __builtin_amdgcn_s_waitcnt(VMCNT(NB));
  if constexpr (SH) {
    if ((int)threadIdx.x < sh.K / 32) sh_sc[threadIdx.x] = (uint8_t)sh_sb;
    // the shared expert's 16 w2 rows (contiguous), in flight during the items
    copy_untracked(sh.w[0] + (size_t)row0 * sh.K, sh_w, 16 * sh.K, wave, nwaves, lane);
  }
  lds_sync();
  if constexpr (SH) {   // act_quant(h_sh) into LDS, read after the items' barrier
    fp8::DecAct<1, DnShape<SH>::THREADS> xa;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(xa.v) / sizeof(xa.v[0])); ++i)
      xa.v[i] = *reinterpret_cast<const uint4*>(sh_h + 16 * min((int)threadIdx.x + DnShape<SH>::THREADS * i,
                                                                 sh.K / 8 - 1));
    fp8::dec_act_quant<1, DnShape<SH>::THREADS>(sh, 1, threadIdx.x, xa, sh_lds);
  }

  f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
  if (slot >= 0) {
    const uint32_t part = j == 0 ? 0u : (uint32_t)F * 2;   // A row 0: hi, row 1: lo, others: zero
    const uint8_t* scale_rows = sc + (size_t)e * 16 * PK;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint32_t aoff =
          (pv[b] && j < 2) ? (uint32_t)e * F * 4 + part + (uint32_t)pi[b] * (PIECE * 2) : (uint32_t)DNZ;
      const float sd = e8m0_to_f32(scale_rows[j * PK + pi[b]]);
#pragma unroll
      for (int s = 0; s < 4; ++s) c = mfma(lds_a(hl, aoff + 16 * s), fp4_codes_to_b(word_of(wd[b], s), sd), c);
    }
  }
  // D[0][j] (hi) and D[1][j] (lo) sit in lane j, registers 0 and 1
  if (lane < 16) vals[e][half][lane] = c[0] + c[1];
  if constexpr (SH) {   // the shared tile's partial tiles, after every wave's copies and quantization
    __builtin_amdgcn_s_waitcnt(0x0F70);   // this wave's w2 row copies
    __syncthreads();
    constexpr int NPV = 8;                // 16 virtual waves over 2k >= 2 waves
    uint32_t bs[NPV][fp8::SH_CPV];
    fp8::dec_wscale<NPV, fp8::SH_CPV>(sh_sc, sh.K, wave, nwaves, lane, bs);
    fp8::dec_mfma_wlds<1, NPV, fp8::SH_CPV>(sh, 1, wave, nwaves, lane, sh_w, bs, sh_lds);
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    const int n = row0 + t;
    float total = 0.0f;
    for (int x = 0; x < k; ++x) {
      float y = 0.0f;
#pragma unroll
      for (int h = 0; h < DN_HALVES; ++h) y = y + vals[x][h][t];
      total = total + y;
    }
    if (routed) routed[n] = total;
    if constexpr (SH) {
      if (out) out[n] = f32_to_bf16(total + round_bf16(fp8::dec_total(sh_lds, 1, sh.K, t, 0)));
    } else {
      if (out) out[n] = f32_to_bf16(addend ? total + bf16_to_f32(addend[n]) : total);
    }
  }
}

}  // namespace

size_t fp4_workspace_bytes(int D, int F, int k) {
  (void)D;
  return ws_offsets((size_t)k * F * sizeof(float)).total;
}

// After the routed workspace: h_sh [F_sh] bf16, then y_sh [D] bf16 (used when the
// shared expert runs in launches of its own).
size_t fp4_shared_region_bytes(int D, int F_sh) {
  return align256((size_t)F_sh * 2) + align256((size_t)D * 2);
}

// The shapes the FP4 launches carry the shared expert for (else it runs first, in
// launches of its own, and its output is the addend).
bool fp4_shared_fused(int D, int F, int k, int F_sh) {
  return D <= fp8::SH_MAX_K && F_sh <= SH_F && k >= 3 && k <= 6 && k * F <= SH_KF;
}

int launch_fp4_decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                      ExpertSource src, const RouterCall* router, int D, int F, int k, float swiglu_limit,
                      const uint16_t* addend, float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                      hipStream_t s, const fp8::SharedWeights* shared = nullptr) {
  CACHALOT_REQUIRE(pool && layout && src.slot_table && x, "moe_decode_fp4: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_fp4: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_fp4: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(src.E >= 1 && src.E <= 1024, "moe_decode_fp4: E=%d outside 1..1024", src.E);
  CACHALOT_REQUIRE(D % 128 == 0 && D >= 128 && D <= MAX_D, "moe_decode_fp4: D=%d must be a multiple of 128 in 128..%d",
                   D, MAX_D);
  CACHALOT_REQUIRE(F % 32 == 0 && F >= 64 && F <= 4096, "moe_decode_fp4: F=%d must be a multiple of 32 in 64..4096",
                   F);
  CACHALOT_REQUIRE(k * F <= MAX_KF, "moe_decode_fp4: k*F=%d exceeds the %d hidden values staged per workgroup",
                   k * F, MAX_KF);
  const WsOffsets wo = ws_offsets((size_t)k * F * sizeof(float));
  const size_t need = wo.total + (shared ? fp4_shared_region_bytes(D, shared->F) : 0);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CACHALOT_ESPACE, "moe_decode_fp4: workspace %zu < %zu bytes", workspace_bytes, need);
  Layout L;
  static const int used[6] = {0, 1, 3, 4, 6, 7};
  int rc = make_layout(layout, 6, used, L, "moe_decode_fp4");
  if (rc) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* hidden = reinterpret_cast<uint16_t*>(ws + wo.hidden);
  int32_t* ws_slots = reinterpret_cast<int32_t*>(ws + wo.slots);
  float* ws_w = reinterpret_cast<float*>(ws + wo.weights);
  if (router) {   // scores only; the gate/up workgroups select the experts
    rc = launch_router_scores(x, router->gate_weight, 1, D, src.E, router->gate_temp, router->score_fn,
                              router->scores, s);
    if (rc) return rc;
    src = route_source(src, *router);
  }
  // the shared expert: carried by the two launches below, or run first with its
  // output as the addend
  const bool sh = shared && fp4_shared_fused(D, F, k, shared->F);
  fp8::DecodeArgs sh_gu{}, sh_dn{};
  if (shared) {
    uint16_t* h_sh = reinterpret_cast<uint16_t*>(ws + wo.total);
    uint16_t* y_sh = h_sh + align256((size_t)shared->F * 2) / 2;
    sh_gu = fp8::DecodeArgs{x, D, {shared->w1, shared->w3}, {shared->s1, shared->s3}, 1, shared->F, D,
                            swiglu_limit, h_sh, shared->F};
    sh_dn = fp8::DecodeArgs{h_sh, shared->F, {shared->w2, shared->w2}, {shared->s2, shared->s2}, 1, D, shared->F,
                            swiglu_limit, y_sh, D};
    if (!sh) {
      rc = fp8::launch_decode(x, shared->w1, shared->s1, shared->w3, shared->s3, shared->w2, shared->s2, 1, D,
                              shared->F, swiglu_limit, h_sh, y_sh, s);
      if (rc) return rc;
      addend = y_sh;
    }
  }
  const int PT = D / PIECE;
  const int nb_gu = ((PT + GU_WAVES - 1) / GU_WAVES + 3) / 4;
  const int xi = (D / 16 + 255) / 256;
  const int n_sh = sh ? shared->F / 8 : 0;
  const dim3 grid_gu(k * (F / 16) + n_sh), block_gu(64 * GU_WAVES);
#define CACHALOT_GU(NBV, XIV)                                                                                \
  if (sh)                                                                                                      \
    hipLaunchKernelGGL((fp4_gate_up_kernel<NBV, XIV, true>), grid_gu, block_gu, 0, s, x, pool, L, src, D, F,   \
                       swiglu_limit, hidden, ws_slots, ws_w, sh_gu, n_sh);                                     \
  else                                                                                                         \
    hipLaunchKernelGGL((fp4_gate_up_kernel<NBV, XIV, false>), grid_gu, block_gu, 0, s, x, pool, L, src, D, F,  \
                       swiglu_limit, hidden, ws_slots, ws_w, sh_gu, n_sh)
  // the smallest instantiated NB >= nb_gu (extra blocks are masked)
  if (xi == 1) {
    if (nb_gu <= 1) CACHALOT_GU(1, 1);
    else if (nb_gu <= 2) CACHALOT_GU(2, 1);
    else if (nb_gu <= 4) CACHALOT_GU(4, 1);
    else if (nb_gu <= 6) CACHALOT_GU(6, 1);
    else CACHALOT_GU(8, 1);
  } else {
    if (nb_gu <= 12) CACHALOT_GU(12, 2);
    else CACHALOT_GU(16, 2);
  }
#undef CACHALOT_GU
  rc = check_launch("fp4_gate_up_kernel");
  if (rc) return rc;
  const int PK = F / PIECE;
  const int nb_dn = ((PK + DN_HALVES - 1) / DN_HALVES + 3) / 4;
  const dim3 grid_dn(D / 16), block_dn(64 * k * DN_HALVES);
#define CACHALOT_DN(NBV)                                                                                        \
  if (sh)                                                                                                         \
    hipLaunchKernelGGL((fp4_down_kernel<NBV, true>), grid_dn, block_dn, 0, s, pool, L, src, ws_slots, D, F, k,    \
                       hidden, nullptr, routed, out, sh_dn);                                                      \
  else                                                                                                            \
    hipLaunchKernelGGL((fp4_down_kernel<NBV, false>), grid_dn, block_dn, 0, s, pool, L, src, ws_slots, D, F, k,   \
                       hidden, addend, routed, out, sh_dn)
  if (nb_dn <= 4) CACHALOT_DN(4);
  else if (nb_dn <= 8) CACHALOT_DN(8);
  else if (nb_dn <= 12) CACHALOT_DN(12);
  else CACHALOT_DN(16);
#undef CACHALOT_DN
  return check_launch("fp4_down_kernel");
}

}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_fp4_workspace_bytes(int D, int F, int k) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX) return 0;
  return cachalot::fp4_workspace_bytes(D, F, k);
}

extern "C" int cachalot_moe_decode_fp4(const uint16_t* x, const uint8_t* pool,
                                       const cachalot_expert_layout* layout, const int32_t* slot_table,
                                       const int32_t* idx, const float* w, int D, int F, int E, int k,
                                       float swiglu_limit, const uint16_t* addend, float* routed, uint16_t* out,
                                       void* workspace, size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(idx && w, "moe_decode_fp4: null pointer");
  decode::ExpertSource src{slot_table, idx, w, E};
  return launch_fp4_decode(x, pool, layout, src, nullptr, D, F, k, swiglu_limit, addend, routed, out, workspace,
                           workspace_bytes, (hipStream_t)stream);
}

extern "C" int cachalot_moe_layer_decode_fp4(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                             int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                             int order, const uint8_t* pool, const cachalot_expert_layout* layout,
                                             const int32_t* slot_table, int D, int F, float swiglu_limit,
                                             const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                             float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                             cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_fp4: null router pointer");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_fp4: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_fp4: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_fp4: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_fp4: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_fp4: invalid topk=%d for %d experts", k, E);
  decode::ExpertSource src{slot_table, nullptr, nullptr, E};
  RouterCall rt{gate_weight, score_fn, gate_temp, scores, {}};
  rt.tail = decode::RouteTail{gate_bias, slot_table, idx_out, w_out, nullptr, nullptr, nullptr, E, k, order, norm,
                              route_scale};
  return launch_fp4_decode(x, pool, layout, src, &rt, D, F, k, swiglu_limit, addend, routed, out, workspace,
                           workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t cachalot_moe_layer_decode_fp4_shared_workspace_bytes(int D, int F, int k, int shared_F) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX || shared_F <= 0) return 0;
  return cachalot::fp4_workspace_bytes(D, F, k) + cachalot::fp4_shared_region_bytes(D, shared_F);
}

extern "C" int cachalot_moe_layer_decode_fp4_shared(
    const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias, int E, int k, int score_fn,
    float gate_temp, float route_scale, int norm, int order, const uint8_t* pool,
    const cachalot_expert_layout* layout, const int32_t* slot_table, int D, int F, float swiglu_limit,
    const uint8_t* shared_w1, const uint8_t* shared_w1_scales, const uint8_t* shared_w3,
    const uint8_t* shared_w3_scales, const uint8_t* shared_w2, const uint8_t* shared_w2_scales, int shared_F,
    int32_t* idx_out, float* w_out, float* scores, float* routed, uint16_t* out, void* workspace,
    size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_fp4_shared: null router pointer");
  CACHALOT_REQUIRE(shared_w1 && shared_w1_scales && shared_w3 && shared_w3_scales && shared_w2 && shared_w2_scales,
                   "moe_layer_decode_fp4_shared: null shared expert pointer");
  CACHALOT_REQUIRE(out, "moe_layer_decode_fp4_shared: out is required (it carries the shared expert)");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_fp4_shared: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(shared_F > 0 && shared_F % 32 == 0 && shared_F <= fp8::DEC_MAX_K && D <= fp8::DEC_MAX_K,
                   "moe_layer_decode_fp4_shared: shared F=%d (a multiple of 32) and D=%d must be at most %d",
                   shared_F, D, fp8::DEC_MAX_K);
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  CACHALOT_REQUIRE(a16(x) && a16(shared_w1) && a16(shared_w3) && a16(shared_w2),
                   "moe_layer_decode_fp4_shared: x and the shared weights must be 16-byte aligned");
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_fp4_shared: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_fp4_shared: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_fp4_shared: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_fp4_shared: invalid topk=%d for %d experts", k,
                   E);
  decode::ExpertSource src{slot_table, nullptr, nullptr, E};
  RouterCall rt{gate_weight, score_fn, gate_temp, scores, {}};
  rt.tail = decode::RouteTail{gate_bias, slot_table, idx_out, w_out, nullptr, nullptr, nullptr, E, k, order, norm,
                              route_scale};
  const fp8::SharedWeights sh{shared_w1, shared_w1_scales, shared_w3, shared_w3_scales, shared_w2, shared_w2_scales,
                              shared_F};
  return launch_fp4_decode(x, pool, layout, src, &rt, D, F, k, swiglu_limit, nullptr, routed, out, workspace,
                           workspace_bytes, (hipStream_t)stream, &sh);
}
