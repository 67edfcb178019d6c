// Decode (one token) over a 2-bit affine g128 expert bank, on the matrix cores.
//
// Reference: src/cachalot/model/expert_affine.py:65-81 (rounding points),
// :117-152 (topk_core: experts summed in route order), moe_layer_metal.py:
// 93-130 (the traced block), mx.quantized_matmul's group formula
// s * sum(x q) + b * sum(x) (MLX qdot, as copied at minimax/codes_qmv.py:86-100).
//
//   q2_gate_up_kernel  one workgroup = one expert x one 16-row tile of W1 and
//                      W3; its four waves split K into quarters.  Every load is
//                      issued before any arithmetic: the lane's codes (lane
//                      group kg of block b takes group 4b + kg of the wave's
//                      quarter, so one load instruction covers whole 128-byte
//                      lines), the tile's scales and biases (one 16-byte load
//                      per thread, staged in LDS) and the token's activations
//                      (staged in LDS in MFMA order with their group sums).
//                      Then 16 v_mfma_f32_16x16x32_bf16 steps per group and
//                      matrix, gate and up sharing each A read; the group
//                      formula is applied per group.  Quarters meet in LDS;
//                      epilogue bf16(g), bf16(u), clamp, h = bf16(silu(g) * u *
//                      w_e), stored group-major in MFMA order.
//   q2_down_kernel     one workgroup = one 16-row tile of W2 for all k experts:
//                      2k waves, wave = (expert, K half).  The k hidden vectors
//                      and the tile's scales are staged in LDS; each expert's row
//                      value is rounded to bf16 (the reference's per-expert
//                      cast) and the experts are summed in route order,
//                      + addend, -> fp32 / bf16.
#include <mutex>

#include "decode_common.h"
#include "fp8_common.h"
#include "mfma_tile.h"
#include "router_launch.h"

namespace cachalot {
namespace {

using namespace decode;
using namespace tile;

constexpr int GU_WAVES = 4;             // K quarters per gate/up workgroup
constexpr int DN_HALVES = 2;            // K halves per expert in the down workgroup
constexpr int MAX_D_GROUPS = 64;        // D <= 8192
constexpr int MAX_F_GROUPS = 32;        // F <= 4096
constexpr int GU_LDS_ZERO = MAX_D_GROUPS * LDS_GROUP_BYTES;
constexpr int DN_LDS_ZERO = KMAX * MAX_F_GROUPS * LDS_GROUP_BYTES;

// Hidden vector of one expert in the workspace: ceil(F / 128) groups, each 128 bf16
// in MFMA order padded to LDS_GROUP_BYTES -- the layout the down kernel stages
// into LDS as is.  Elements from F up to the group boundary are zero.
__host__ __device__ inline int hidden_stride(int F) { return (F + GROUP - 1) / GROUP * (LDS_GROUP_BYTES / 2); }
__device__ __forceinline__ int hidden_index(int n) { return (n >> 7) * (LDS_GROUP_BYTES / 2) + mfma_index(n & 127); }

// 16 MFMA steps over one 128-code group and two matrices sharing A.
__device__ __forceinline__ void group_steps2(const uint8_t* lds, uint32_t aoff, const uint4 (&wa)[2],
                                             const uint4 (&wb)[2], f32x4_t& ca, f32x4_t& cb) {
  ca = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  cb = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const bf16x8_t a = lds_a(lds, aoff + 16 * s);
    const uint32_t w0 = word_of(wa[s >> 3], (s >> 1) & 3);
    const uint32_t w1 = word_of(wb[s >> 3], (s >> 1) & 3);
    if (s & 1) {
      ca = mfma(a, q2_codes_to_b<1>(w0), ca);
      cb = mfma(a, q2_codes_to_b<1>(w1), cb);
    } else {
      ca = mfma(a, q2_codes_to_b<0>(w0), ca);
      cb = mfma(a, q2_codes_to_b<0>(w1), cb);
    }
  }
}

__device__ __forceinline__ f32x4_t group_steps1(const uint8_t* lds, uint32_t aoff, const uint4 (&wa)[2]) {
  f32x4_t ca = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const bf16x8_t a = lds_a(lds, aoff + 16 * s);
    const uint32_t w0 = word_of(wa[s >> 3], (s >> 1) & 3);
    if (s & 1) ca = mfma(a, q2_codes_to_b<1>(w0), ca);
    else ca = mfma(a, q2_codes_to_b<0>(w0), ca);
  }
  return ca;
}

// Lane group kg of block b of a wave owning groups [first, first + GW) takes
// group first + 4b + kg (valid when 4b + kg < GW and below `groups`).
template <int NB>
__device__ __forceinline__ void lane_groups(int first, int GW, int groups, int kg, int (&gi)[NB], bool (&gv)[NB]) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int within = 4 * b + kg;
    const int G = first + within;
    gv[b] = within < GW && G < groups;
    gi[b] = min(G, groups - 1);
  }
}

// grid.x = k * F / 16.  NB = ceil(ceil(D/128 / 4) / 4) groups per lane group;
// XI = ceil(D / 4096) activation items (and scale pieces) per thread.
template <int NB, int XI>
__global__ void __launch_bounds__(64 * GU_WAVES) q2_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ pool, Layout L, ExpertSource src, int D, int F,
    float limit, uint16_t* __restrict__ hp, int32_t* __restrict__ ws_slots, float* __restrict__ ws_w) {
  __shared__ __align__(16) uint8_t xm[GU_LDS_ZERO + LDS_ZERO_BYTES];
  __shared__ __align__(16) uint16_t sc[4 * 16 * MAX_D_GROUPS];   // s1, b1, s3, b3 of the tile's rows
  __shared__ float xs[MAX_D_GROUPS];
  __shared__ float red[GU_WAVES][2][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int GT = D / GROUP;
  const int tiles = F / 16;
  const int e = blockIdx.x / tiles;
  const int tile = blockIdx.x - e * tiles;
  const int row0 = tile * 16;
  __shared__ int top_i[GU_WAVES][KMAX];
  __shared__ float top_v[GU_WAVES][KMAX], top_w[GU_WAVES][KMAX];
  __shared__ int top_s[GU_WAVES][KMAX];
  const int slot = route_slot(src, ws_slots, e, top_i[wave], top_v[wave], top_s[wave]);
  if ((src.idx || src.scores) && tile == 0 && threadIdx.x == 0) ws_slots[e] = slot;   // read by the down kernel
  uint16_t* hout = hp + (size_t)e * hidden_stride(F);
  const int tail = (F + GROUP - 1) / GROUP * GROUP - F;
  if (tile == 0 && (int)threadIdx.x < tail) hout[hidden_index(F + threadIdx.x)] = 0;
  if (slot < 0) {   // the expert has no slot: its hidden rows are zero
    if (threadIdx.x < 16) {
      hout[hidden_index(row0 + threadIdx.x)] = 0;
      route_finish(src, ws_w, e, tile, top_v[0], top_w[0], top_i[0], blockIdx.x == 0);
    }
    return;
  }
  const uint8_t* base = pool + (int64_t)slot * L.record_bytes;
  const int j = lane & 15, kg = lane >> 4;
  const int row = row0 + j;
  int gi[NB];
  bool gv[NB];
  const int GW = (GT + GU_WAVES - 1) / GU_WAVES;
  lane_groups<NB>(wave * GW, GW, GT, kg, gi, gv);

  // 1. the lane's codes (both matrices)
  uint4 wg[NB][2], wu[NB][2];
  {
    const uint4* r1 = reinterpret_cast<const uint4*>(base + L.off[0]) + (size_t)row * GT * 2;
    const uint4* r3 = reinterpret_cast<const uint4*>(base + L.off[6]) + (size_t)row * GT * 2;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      wg[b][0] = r1[2 * gi[b]];
      wg[b][1] = r1[2 * gi[b] + 1];
      wu[b][0] = r3[2 * gi[b]];
      wu[b][1] = r3[2 * gi[b] + 1];
    }
  }
  // 2. the tile's scales and biases (4 tensors x 16 rows x GT bf16, each a contiguous run) into LDS
  {
    const int run = 32 * GT;
    const int64_t toff[4] = {L.off[1], L.off[2], L.off[7], L.off[8]};
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma_to_lds(base + toff[q] + (int64_t)row0 * GT * 2, reinterpret_cast<uint8_t*>(sc) + q * run, run,
                 (wave + q) & 3, GU_WAVES, lane);
  }
  // 3. the activations: 16 values per item
  uint4 xa[XI][2];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int t = min((int)threadIdx.x + 256 * i, D / 16 - 1);
    const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)t * 16);
    xa[i][0] = p[0];
    xa[i][1] = p[1];
  }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int t = threadIdx.x + 256 * i;
    uint4 lo, hi;
    pairs_mfma(xa[i][0].x, xa[i][0].y, lo.x, lo.y);
    pairs_mfma(xa[i][0].z, xa[i][0].w, lo.z, lo.w);
    pairs_mfma(xa[i][1].x, xa[i][1].y, hi.x, hi.y);
    pairs_mfma(xa[i][1].z, xa[i][1].w, hi.z, hi.w);
    const float sum = sum8_lanes(sum_bf16x8(lo) + sum_bf16x8(hi));
    if (t < D / 16) {
      uint4* d = reinterpret_cast<uint4*>(xm + (t >> 3) * LDS_GROUP_BYTES + (t & 7) * 32);
      d[0] = lo;
      d[1] = hi;
      if ((t & 7) == 0) xs[t >> 3] = sum;
    }
  }
  if (threadIdx.x < LDS_ZERO_BYTES / 16)
    reinterpret_cast<uint4*>(xm + GU_LDS_ZERO)[threadIdx.x] = make_uint4(0, 0, 0, 0);
  wait_vmem();
  __syncthreads();

  const uint16_t* s1 = sc;
  const uint16_t* b1 = sc + 16 * GT;
  const uint16_t* s3 = sc + 32 * GT;
  const uint16_t* b3 = sc + 48 * GT;
  float accg = 0.0f, accu = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint32_t aoff = (gv[b] && j == 4 * kg) ? (uint32_t)gi[b] * LDS_GROUP_BYTES : (uint32_t)GU_LDS_ZERO;
    f32x4_t cg, cu;
    group_steps2(xm, aoff, wg[b], wu[b], cg, cu);
    const float gs = gv[b] ? xs[gi[b]] : 0.0f;
    const int si = j * GT + gi[b];
    accg = accg + (scale_bits_to_f32(s1[si], L.f16) * cg[0] + scale_bits_to_f32(b1[si], L.f16) * gs);
    accu = accu + (scale_bits_to_f32(s3[si], L.f16) * cu[0] + scale_bits_to_f32(b3[si], L.f16) * gs);
  }
  accg = sum_lane_groups(accg);
  accu = sum_lane_groups(accu);
  if (lane < 16) {
    red[wave][0][lane] = accg;
    red[wave][1][lane] = accu;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const float wexp = route_finish(src, ws_w, e, tile, top_v[0], top_w[0], top_i[0], blockIdx.x == 0);
    const int t = threadIdx.x;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int w = 0; w < GU_WAVES; ++w) {
      g = g + red[w][0][t];
      u = u + red[w][1][t];
    }
    g = round_bf16(g);
    u = round_bf16(u);
    if (limit > 0.0f) {
      u = fminf(fmaxf(u, -limit), limit);
      g = fminf(g, limit);
    }
    const float h = (silu_f32(g) * u) * wexp;
    hout[hidden_index(row0 + t)] = f32_to_bf16(h);
  }
}

// grid.x = D / 16; block = 64 * k * DN_HALVES threads.  NB = ceil(GK / 8) with
// GK = ceil(F / 128) groups per lane group.
template <int NB>
__global__ void __launch_bounds__(64 * KMAX * DN_HALVES) q2_down_kernel(
    const uint8_t* __restrict__ pool, Layout L, const int32_t* __restrict__ ws_slots, int D, int F, int k,
    const uint16_t* __restrict__ hp, const uint16_t* __restrict__ addend, float* __restrict__ routed,
    uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint8_t hm[DN_LDS_ZERO + LDS_ZERO_BYTES];
  __shared__ __align__(16) uint16_t sc[KMAX * 2 * 16 * MAX_F_GROUPS];   // per expert: s2, b2 of the tile's rows
  __shared__ float hsum[KMAX * MAX_F_GROUPS];
  __shared__ float vals[KMAX][DN_HALVES][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int GK = (F + GROUP - 1) / GROUP;   // groups per W2 row (the last may be partial)
  const int e = wave / DN_HALVES;
  const int half = wave - e * DN_HALVES;
  const int row0 = blockIdx.x * 16;
  const int j = lane & 15, kg = lane >> 4;
  const int slot = ws_slots[e];
  const int GW = (GK + DN_HALVES - 1) / DN_HALVES;
  int gi[NB];
  bool gv[NB];
  lane_groups<NB>(half * GW, GW, GK, kg, gi, gv);

  // 1. the lane's codes
  uint4 wd[NB][2];
  if (slot >= 0) {
    const uint4* r2 =
        reinterpret_cast<const uint4*>(pool + (int64_t)slot * L.record_bytes + L.off[3]) + (size_t)(row0 + j) * GK * 2;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      wd[b][0] = r2[2 * gi[b]];
      wd[b][1] = r2[2 * gi[b] + 1];
    }
  }
  // 2. the hidden vectors (already in LDS layout) and, per expert, the tile's
  //    scales and biases (two contiguous runs of 16 rows x GK bf16) into LDS
  dma_to_lds(hp, hm, k * GK * LDS_GROUP_BYTES, wave, nwaves, lane);
  {
    const int run = 32 * GK;
    for (int r = wave; r < 2 * k; r += nwaves) {
      const int re = r >> 1;
      const int ps = max(ws_slots[re], 0);   // a missing expert's rows are never used
      dma_to_lds(pool + (int64_t)ps * L.record_bytes + ((r & 1) ? L.off[5] : L.off[4]) + (int64_t)row0 * GK * 2,
                 reinterpret_cast<uint8_t*>(sc) + r * run, run, 0, 1, lane);
    }
  }
  if (threadIdx.x < LDS_ZERO_BYTES / 16)
    reinterpret_cast<uint4*>(hm + DN_LDS_ZERO)[threadIdx.x] = make_uint4(0, 0, 0, 0);
  wait_vmem();
  __syncthreads();
  // group sums of the hidden vectors: 16 chunks of 8 values per group
  {
    const int chunks = k * GK * 16;
    for (int c0 = 0; c0 < chunks; c0 += blockDim.x) {
      const int c = c0 + threadIdx.x;
      const int cc = min(c, chunks - 1);
      const uint4 v = *reinterpret_cast<const uint4*>(hm + (cc >> 4) * LDS_GROUP_BYTES + (cc & 15) * 16);
      const float sum = row16_sum(sum_bf16x8(v));
      if (c < chunks && (c & 15) == 0) hsum[c >> 4] = sum;
    }
  }
  __syncthreads();

  float acc = 0.0f;
  if (slot >= 0) {
    const uint16_t* s2 = sc + e * 32 * GK;
    const uint16_t* b2 = s2 + 16 * GK;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint32_t aoff =
          (gv[b] && j == 4 * kg) ? (uint32_t)(e * GK + gi[b]) * LDS_GROUP_BYTES : (uint32_t)DN_LDS_ZERO;
      const f32x4_t c = group_steps1(hm, aoff, wd[b]);
      const float gs = gv[b] ? hsum[e * GK + gi[b]] : 0.0f;
      const int si = j * GK + gi[b];
      acc = acc + (scale_bits_to_f32(s2[si], L.f16) * c[0] + scale_bits_to_f32(b2[si], L.f16) * gs);
    }
  }
  acc = sum_lane_groups(acc);
  if (lane < 16) vals[e][half][lane] = acc;
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    const int n = row0 + t;
    float total = 0.0f;
    for (int x = 0; x < k; ++x) {
      float y = 0.0f;
#pragma unroll
      for (int h = 0; h < DN_HALVES; ++h) y = y + vals[x][h][t];
      total = total + round_bf16(y);
    }
    if (routed) routed[n] = total;
    if (out) out[n] = f32_to_bf16(addend ? total + bf16_to_f32(addend[n]) : total);
  }
}

}  // namespace

// [decode layout (counters, slots, weights, bf16 hidden)]
// [matrix-core path: hidden plane blocks, k x ceil(F/128) x 320 B][x plane blocks, ceil(D/128) x 320 B]
static size_t xplanes_bytes(int D) { return align256((size_t)(D + 127) / 128 * 320); }
static size_t hplanes_bytes(int F, int k) { return align256((size_t)k * ((F + 127) / 128) * 320); }
size_t q2_workspace_bytes(int D, int F, int k) {
  return ws_offsets((size_t)k * hidden_stride(F) * sizeof(uint16_t)).total + hplanes_bytes(F, k) + xplanes_bytes(D);
}

// Validates, then launches [router + top-k tail], gate/up and down on stream s.
// With `router` the experts come from the router tail, else from src.idx / src.w.

bool q2mx_supported(int D, int F, int k);
bool q2mx_shared_supported(int D, int F_sh);
int launch_q2mx_decode(const uint16_t* x, bool planes_ready, uint8_t* xplanes, const uint8_t* pool,
                       const Layout& L, const ExpertSource& src, int32_t* ws_slots, float* ws_w, int D, int F,
                       int k, float limit, const uint16_t* addend, float* routed, uint16_t* out, uint8_t* hid,
                       hipStream_t s, const fp8::DecodeArgs* sh_gu, const fp8::DecodeArgs* sh_dn);
using SharedFp8 = fp8::SharedWeights;
// After the routed workspace: h_sh [F] bf16, then y_sh [D] bf16 (used when the
// shared expert runs in launches of its own).
static size_t shared_region_bytes(int D, int F_sh) { return align256((size_t)F_sh * 2) + align256((size_t)D * 2); }

// The bf16 kernels stay selectable (CACHALOT_DECODE_BF16=1) for comparison.
static bool bf16_requested() {
  const char* env = getenv("CACHALOT_DECODE_BF16");
  return env && env[0] == '1';
}

int launch_q2_decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                     ExpertSource src, const RouterCall* router, int D, int F, int k, int group, float swiglu_limit,
                     const uint16_t* addend, float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                     hipStream_t s, const SharedFp8* shared = nullptr) {
  CACHALOT_REQUIRE(pool && layout && src.slot_table && x, "moe_decode_q2: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_q2: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_q2: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(src.E >= 1 && src.E <= 1024, "moe_decode_q2: E=%d outside 1..1024", src.E);
  CACHALOT_REQUIRE(group == GROUP, "moe_decode_q2: group_size %d (the bank format uses 128)", group);
  CACHALOT_REQUIRE(D % GROUP == 0 && D >= GROUP && D <= GROUP * MAX_D_GROUPS,
                   "moe_decode_q2: D=%d must be a multiple of 128 in 128..8192", D);
  CACHALOT_REQUIRE(F % 16 == 0 && F >= 64 && F <= GROUP * MAX_F_GROUPS,
                   "moe_decode_q2: F=%d must be a multiple of 16 in 64..4096", F);
  const WsOffsets wo = ws_offsets((size_t)k * hidden_stride(F) * sizeof(uint16_t));
  const size_t need = q2_workspace_bytes(D, F, k) + (shared ? shared_region_bytes(D, shared->F) : 0);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CACHALOT_ESPACE, "moe_decode_q2: workspace %zu < %zu bytes", workspace_bytes, need);
  Layout L;
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  int rc = make_layout(layout, 9, used, L, "moe_decode_q2");
  if (rc) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* hp = reinterpret_cast<uint16_t*>(ws + wo.hidden);
  int32_t* ws_slots = reinterpret_cast<int32_t*>(ws + wo.slots);
  float* ws_w = reinterpret_cast<float*>(ws + wo.weights);
  const bool mx = q2mx_supported(D, F, k) && !bf16_requested();
  uint8_t* xplanes = ws + wo.total + hplanes_bytes(F, k);
  if (router && mx) {   // scores only; the gate/up workgroups select the experts
    rc = launch_router_scores(x, router->gate_weight, 1, D, src.E, router->gate_temp, router->score_fn,
                              router->scores, s, nullptr, mx ? xplanes : nullptr);
    if (rc) return rc;
    src = route_source(src, *router);
  } else if (router) {
    RouteTail tail = router->tail;
    tail.ws_slots = ws_slots;
    tail.ws_w = ws_w;
    tail.counter = &reinterpret_cast<Counters*>(ws + wo.counter)->route_done;
    rc = launch_router_scores(x, router->gate_weight, 1, D, src.E, router->gate_temp, router->score_fn,
                              router->scores, s, &tail);
    if (rc) return rc;
    src.idx = nullptr;
    src.w = nullptr;
  }
  if (shared) {
    uint16_t* h_sh = reinterpret_cast<uint16_t*>(ws + q2_workspace_bytes(D, F, k));
    uint16_t* y_sh = h_sh + align256((size_t)shared->F * 2) / 2;
    if (mx && q2mx_shared_supported(D, shared->F)) {   // carried by the routed launches
      const fp8::DecodeArgs gu{x, D, {shared->w1, shared->w3}, {shared->s1, shared->s3}, 1, shared->F, D,
                               swiglu_limit, h_sh, shared->F};
      const fp8::DecodeArgs dn{h_sh, shared->F, {shared->w2, shared->w2}, {shared->s2, shared->s2}, 1, D,
                               shared->F, swiglu_limit, y_sh, D};
      return launch_q2mx_decode(x, router != nullptr, xplanes, pool, L, src, ws_slots, ws_w, D, F, k,
                                swiglu_limit, nullptr, routed, out, ws + wo.total, s, &gu, &dn);
    }
    // its own two launches ahead of the experts, y_sh as the addend
    rc = fp8::launch_decode(x, shared->w1, shared->s1, shared->w3, shared->s3, shared->w2, shared->s2, 1, D,
                            shared->F, swiglu_limit, h_sh, y_sh, s);
    if (rc) return rc;
    addend = y_sh;
  }
  if (mx)
    return launch_q2mx_decode(x, router != nullptr, xplanes, pool, L, src, ws_slots, ws_w, D, F, k, swiglu_limit,
                              addend, routed, out, ws + wo.total, s, nullptr, nullptr);
  const int GT = D / GROUP;
  const int nb_gu = ((GT + GU_WAVES - 1) / GU_WAVES + 3) / 4;
  const int xi = (D / 16 + 255) / 256;
  const dim3 grid_gu(k * (F / 16)), block_gu(64 * GU_WAVES);
#define CACHALOT_GU(NBV, XIV)                                                                                  \
  hipLaunchKernelGGL((q2_gate_up_kernel<NBV, XIV>), grid_gu, block_gu, 0, s, x, pool, L, src, D, F, swiglu_limit, \
                     hp, ws_slots, ws_w)
  if (xi == 1) {
    switch (nb_gu) {
      case 1: CACHALOT_GU(1, 1); break;
      default: CACHALOT_GU(2, 1); break;
    }
  } else {
    switch (nb_gu) {
      case 3: CACHALOT_GU(3, 2); break;
      default: CACHALOT_GU(4, 2); break;
    }
  }
#undef CACHALOT_GU
  rc = check_launch("q2_gate_up_kernel");
  if (rc) return rc;
  const int GK = (F + GROUP - 1) / GROUP;
  const int nb_dn = (GK + 7) / 8;
  const dim3 grid_dn(D / 16), block_dn(64 * k * DN_HALVES);
#define CACHALOT_DN(NBV)                                                                                   \
  hipLaunchKernelGGL((q2_down_kernel<NBV>), grid_dn, block_dn, 0, s, pool, L, ws_slots, D, F, k, hp, addend, \
                     routed, out)
  switch (nb_dn) {
    case 1: CACHALOT_DN(1); break;
    case 2: CACHALOT_DN(2); break;
    case 3: CACHALOT_DN(3); break;
    default: CACHALOT_DN(4); break;
  }
#undef CACHALOT_DN
  return check_launch("q2_down_kernel");
}

}  // namespace cachalot

extern "C" size_t cachalot_moe_decode_q2_workspace_bytes(int D, int F, int k) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX) return 0;
  return cachalot::q2_workspace_bytes(D, F, k);
}

extern "C" int cachalot_moe_decode_q2(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                                      const int32_t* slot_table, const int32_t* idx, const float* w, int D, int F,
                                      int E, int k, int group, float swiglu_limit, const uint16_t* addend,
                                      float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                      cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(idx && w, "moe_decode_q2: null pointer");
  decode::ExpertSource src{slot_table, idx, w, E};
  return launch_q2_decode(x, pool, layout, src, nullptr, D, F, k, group, swiglu_limit, addend, routed, out,
                          workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cachalot_moe_layer_decode_q2(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                            int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                            int order, const uint8_t* pool, const cachalot_expert_layout* layout,
                                            const int32_t* slot_table, int D, int F, int group, float swiglu_limit,
                                            const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                            float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                            cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_q2: null router pointer");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_q2: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_q2: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_q2: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_q2: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_q2: invalid topk=%d for %d experts", k, E);
  decode::ExpertSource src{slot_table, nullptr, nullptr, E};
  RouterCall rt{gate_weight, score_fn, gate_temp, scores, {}};
  rt.tail = decode::RouteTail{gate_bias, slot_table, idx_out, w_out, nullptr, nullptr, nullptr, E, k, order, norm,
                              route_scale};
  return launch_q2_decode(x, pool, layout, src, &rt, D, F, k, group, swiglu_limit, addend, routed, out, workspace,
                          workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t cachalot_moe_layer_decode_q2_shared_workspace_bytes(int D, int F, int k, int shared_F) {
  if (D <= 0 || F <= 0 || k <= 0 || k > cachalot::decode::KMAX || shared_F <= 0) return 0;
  return cachalot::q2_workspace_bytes(D, F, k) + cachalot::shared_region_bytes(D, shared_F);
}

extern "C" int cachalot_moe_layer_decode_q2_shared(
    const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias, int E, int k, int score_fn,
    float gate_temp, float route_scale, int norm, int order, const uint8_t* pool,
    const cachalot_expert_layout* layout, const int32_t* slot_table, int D, int F, int group, float swiglu_limit,
    const uint8_t* shared_w1, const uint8_t* shared_w1_scales, const uint8_t* shared_w3,
    const uint8_t* shared_w3_scales, const uint8_t* shared_w2, const uint8_t* shared_w2_scales, int shared_F,
    int32_t* idx_out, float* w_out, float* scores, float* routed, uint16_t* out, void* workspace,
    size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_q2_shared: null router pointer");
  CACHALOT_REQUIRE(shared_w1 && shared_w1_scales && shared_w3 && shared_w3_scales && shared_w2 && shared_w2_scales,
                   "moe_layer_decode_q2_shared: null shared expert pointer");
  CACHALOT_REQUIRE(out, "moe_layer_decode_q2_shared: out is required (it carries the shared expert)");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_q2_shared: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(shared_F > 0 && shared_F % 32 == 0 && shared_F <= fp8::DEC_MAX_K && D <= fp8::DEC_MAX_K,
                   "moe_layer_decode_q2_shared: shared F=%d (a multiple of 32) and D=%d must be at most %d", shared_F,
                   D, fp8::DEC_MAX_K);
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  CACHALOT_REQUIRE(a16(x) && a16(shared_w1) && a16(shared_w3) && a16(shared_w2),
                   "moe_layer_decode_q2_shared: x and the shared weights must be 16-byte aligned");
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_q2_shared: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_q2_shared: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_q2_shared: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_q2_shared: invalid topk=%d for %d experts", k,
                   E);
  decode::ExpertSource src{slot_table, nullptr, nullptr, E};
  RouterCall rt{gate_weight, score_fn, gate_temp, scores, {}};
  rt.tail = decode::RouteTail{gate_bias, slot_table, idx_out, w_out, nullptr, nullptr, nullptr, E, k, order, norm,
                              route_scale};
  const SharedFp8 sh{shared_w1, shared_w1_scales, shared_w3, shared_w3_scales, shared_w2, shared_w2_scales, shared_F};
  return launch_q2_decode(x, pool, layout, src, &rt, D, F, k, group, swiglu_limit, nullptr, routed, out, workspace,
                          workspace_bytes, (hipStream_t)stream, &sh);
}

// ------------------------------------------------- decode with no allocation ---
// cachalot_moe_layer_decode_q2_static: cachalot_moe_layer_decode_q2 with its
// workspace in a file-scope device array instead of a caller's buffer, for callers
// that cannot allocate (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc).  Each GPU the library runs on holds its own copy of the array
// (STATIC_SCRATCH_BYTES) until the process ends; every call on one GPU shares it,
// so calls that overlap on one GPU race.  Nothing here allocates: the array's
// device address comes from hipGetSymbolAddress, once per device, and the kernels
// receive that address exactly as they receive a caller's workspace.
//
// What must start at zero: the counters at the head of the workspace.  The loader
// zero-fills the array, the first call on each device clears it once more with a
// fill kernel on the caller's stream, and every call leaves the counters at zero.
namespace cachalot {
namespace {
constexpr size_t STATIC_SCRATCH_BYTES = 256 * 1024;
constexpr int STATIC_MAX_DEVICES = 64;
}  // namespace
}  // namespace cachalot

static __device__ __align__(256) uint8_t scratch[cachalot::STATIC_SCRATCH_BYTES];

namespace cachalot {
namespace {

std::mutex g_scratch_mu;
uint8_t* g_scratch[STATIC_MAX_DEVICES] = {};

__global__ void __launch_bounds__(256) scratch_clear_kernel(uint4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

// The current device's copy of `scratch` (device address), set up on first use.
int static_scratch(uint8_t** out, hipStream_t s) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= STATIC_MAX_DEVICES)
    return fail(CACHALOT_EHIP, "moe_layer_decode_q2_static: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(CACHALOT_EHIP, "moe_layer_decode_q2_static: hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(err));
    hipLaunchKernelGGL(scratch_clear_kernel, dim3(64), dim3(256), 0, s, static_cast<uint4*>(p),
                       STATIC_SCRATCH_BYTES / 16);
    const int rc = check_launch("scratch_clear_kernel");
    if (rc) return rc;
    g_scratch[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch[dev];
  return CACHALOT_OK;
}

}  // namespace
}  // namespace cachalot

extern "C" size_t cachalot_moe_layer_decode_q2_static_max_bytes(void) { return cachalot::STATIC_SCRATCH_BYTES; }

extern "C" int cachalot_moe_layer_decode_q2_static(const uint16_t* x, const uint16_t* gate_weight,
                                                   const float* gate_bias, int E, int k, int score_fn,
                                                   float gate_temp, float route_scale, int norm, int order,
                                                   const uint8_t* pool, const cachalot_expert_layout* layout,
                                                   const int32_t* slot_table, int D, int F, int group,
                                                   float swiglu_limit, const uint16_t* addend, int32_t* idx_out,
                                                   float* w_out, float* scores, float* routed, uint16_t* out,
                                                   cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(D > 0 && F > 0 && k >= 1 && k <= decode::KMAX,
                   "moe_layer_decode_q2_static: D=%d F=%d k=%d", D, F, k);
  const size_t need = q2_workspace_bytes(D, F, k);
  if (need > STATIC_SCRATCH_BYTES)
    return fail(CACHALOT_ESPACE,
                "moe_layer_decode_q2_static: D=%d F=%d k=%d needs %zu bytes of scratch, the static array holds %zu "
                "(use cachalot_moe_layer_decode_q2 with a workspace)",
                D, F, k, need, STATIC_SCRATCH_BYTES);
  uint8_t* ws = nullptr;
  const int rc = static_scratch(&ws, (hipStream_t)stream);
  if (rc) return rc;
  return cachalot_moe_layer_decode_q2(x, gate_weight, gate_bias, E, k, score_fn, gate_temp, route_scale, norm, order,
                                      pool, layout, slot_table, D, F, group, swiglu_limit, addend, idx_out, w_out,
                                      scores, routed, out, ws, STATIC_SCRATCH_BYTES, stream);
}
