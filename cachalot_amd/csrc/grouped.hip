// Expert-major (grouped) MoE for many tokens: prefill chunks and batched decode.
//
// Reference: src/cachalot/model/moe_prefill_grouped.py -- dispatch :199-245
// (assignments per expert, tokens ascending, route slot kept), per-expert
// forward :420-467 (affine_expert_forward_batched, expert_affine.py:84-99;
// routed_expert_forward_sgmm / _batched, fp4_sgmm_metal.py:318-333,
// moe_prefill_batched.py:31-61), combine :526-545 (slot 0 + ... + slot k-1 in
// fp32, then the dtype cast).  Rounding points of every path: g = bf16(x W1),
// u = bf16(x W3), h = bf16(silu(min(g, L)) * clip(u, +-L) * w), y = bf16(h W2).
//
//   permute_scatter_kernel (or permute_small_kernel up to 1024 routes)
//       rows grouped by expert (ascending), tokens ascending inside an expert:
//       offsets [E+1], row_token, row_slot, row_w.  The scatter runs one
//       workgroup per expert over all T*k routes with ballot compaction, so
//       the order is the reference's by construction.
//   tile_list_kernel   (expert, first row) of every MT-row tile.
//   grouped_gate_up_kernel<KIND, MT>
//       one workgroup = one M tile (MT rows of one expert, gathered from x by
//       row_token) x 64 rows of W1 and W3; wave w owns 16 weight rows; K in
//       chunks of 128 (one 2-bit group, four FP4 blocks) with the A chunk
//       double-buffered in LDS and the next chunk's codes prefetched in
//       registers.  v_mfma_f32_16x16x32_bf16 with A = activations, B = codes
//       converted to bf16 (2-bit: integer codes, group formula applied per
//       chunk as s * C + b * sum(x); FP4: E2M1 x 2^e, exact).  Epilogue writes
//       h = bf16(silu(min(bf16 g, L)) * clip(bf16 u) * w) row-major [rows, F].
//   grouped_down_kernel<KIND, MT>
//       same tiling over W2 with A = h rows; y = bf16(h W2) goes straight to
//       its (token, route slot) place: y [T, k, D] bf16.
//   combine_kernel     out[t] = bf16(0 + y[t,0] + ... + y[t,k-1] (+ addend));
//                      combine8_kernel the same with 16-byte accesses.
// The grouped kernels also take the other affine widths (aff_kind<BITS, G>: 3- and
// 4-bit codes, groups of 32 / 64 / 128, 2-bit codes in groups of 32 / 64), with the
// codes read per step and the group formula applied per group (see chunk_mma_aff).
// FP4, 2-bit g128 and (2-bit g64, 3- / 4-bit g64 / g128) affine prefill go to the
// block-scaled kernels of prefill_mx.hip and prefill_affine_mx.hip; these kernels take
// groups of 32, the other shapes and CACHALOT_PREFILL_BF16=1.
#include "decode_common.h"
#include "mfma_tile.h"
#include "permute_small.h"

#include <algorithm>

namespace cachalot {

}  // namespace cachalot
extern "C" int cachalot_permute(const int32_t* idx, const float* w, int T, int k, int E, int32_t* offsets,
                                int32_t* row_token, int32_t* row_slot, float* row_w, cachalot_stream_t stream);
namespace cachalot {

// matrix-core batched decode (decode_q2_mx.hip)
bool q2mx_supported(int D, int F, int k);
int launch_q2mx_batched(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L,
                        const int32_t* slot_table, const int32_t* offsets, int E, int4* recs, int32_t* n_recs,
                        int max_active, const int32_t* row_token, const int32_t* row_slot, const float* row_w, int D,
                        int F, int k, float limit, uint8_t* hid, uint8_t* xplanes, uint16_t* y, hipStream_t s,
                        const int32_t* ridx, const float* rw);

// FP4 prefill on the block-scaled matrix cores (prefill_mx.hip)
size_t prefill_mx_ws_bytes(int T, int k, int D, int F);
bool prefill_mx_supported(int D, int F, const decode::Layout& L);
int prefill_mx_mt();
bool prefill_mx_aff_supported(int bits, int group, int D, int F, const decode::Layout& L);
int launch_prefill_mx_aff(int bits, int group, const uint16_t* x, int T, const uint8_t* pool,
                          const decode::Layout& L, const int32_t* slot_table, const int32_t* offsets,
                          const int2* tiles, const int32_t* tiles_n, int max_tiles, const int32_t* row_token,
                          const int32_t* row_slot, const float* row_w, int D, int F, int k, float limit, uint8_t* ws,
                          uint16_t* y, hipStream_t s);
int launch_prefill_mx(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L,
                      const int32_t* slot_table, const int32_t* offsets, const int2* tiles, const int32_t* tiles_n,
                      int max_tiles, const int32_t* row_token, const int32_t* row_slot, const float* row_w, int D,
                      int F, int k, float limit, uint8_t* ws, uint16_t* y, hipStream_t s);
bool prefill_mx_q2_supported(int D, int F, const decode::Layout& L);
int launch_prefill_mx_q2(const uint16_t* x, int T, const uint8_t* pool, const decode::Layout& L,
                         const int32_t* slot_table, const int32_t* offsets, const int2* tiles,
                         const int32_t* tiles_n, int max_tiles, const int32_t* row_token, const int32_t* row_slot,
                         const float* row_w, int D, int F, int k, float limit, uint8_t* ws, uint16_t* y,
                         hipStream_t s);

namespace {

using namespace decode;
using namespace tile;

constexpr int KIND_Q2 = 0;
constexpr int KIND_FP4 = 1;
// Affine banks of the other widths (3- and 4-bit codes, groups of 32 / 64 / 128, 2-bit
// codes in groups of 32 / 64): KIND_AFF + 10 bits + group / 32.  Their K chunk of 128
// holds 128 / G groups; a step of the bf16 matrix cores covers 32 contiguous codes
// (lane group kg: codes 32 s + 8 kg ..), so a group is G / 32 whole steps and its
// formula s * sum(x q) + b * sum(x) is applied after its last step.
constexpr int KIND_AFF = 100;
template <int BITS, int G>
constexpr int aff_kind = KIND_AFF + 10 * BITS + G / 32;
constexpr bool is_aff(int kind) { return kind >= KIND_AFF; }
constexpr int aff_bits(int kind) { return (kind - KIND_AFF) / 10; }
constexpr int aff_group(int kind) { return ((kind - KIND_AFF) % 10) * 32; }
constexpr int NT = 64;                 // weight rows per workgroup (4 waves x 16)
constexpr int KC = 128;                // K chunk
constexpr int A_ROW_BYTES = 272;       // one staged A row: 128 bf16 + 16 bytes padding
constexpr int MAX_GROUPS = 64;         // K <= 8192
constexpr int PERMUTE_THREADS = 1024;
constexpr int ZERO_WORDS = 16;         // 64 zero bytes at offset 128 of the workspace

// ------------------------------------------------------------------ permute ---
// One 1024-thread workgroup per expert e, keeping the routes that chose e in route
// order.  Workgroup E collects the routes whose id lies outside [0, E) into rows
// [offsets[E], n), in route order, with weight 0: the dropped routes, whose y rows
// drop_zero_kernel clears.  Wave w owns the w-th of 16 contiguous segments of the
// routes: it counts its hits and the routes of lower experts (ballots, no barrier);
// one barrier gives the expert's first row -- offsets[e], which the workgroup writes
// (workgroup E: offsets[E], the valid routes) -- and each segment the hits of the
// segments before it, and the wave walks its segment again writing rows.  (Config 3, 24,576 routes: 64.5 us with one 256-thread workgroup stepping
// through all routes, 29.9 us so; 512- and 256-thread workgroups 35.8 / 50.3 us.)
constexpr int SCATTER_THREADS = 1024;
__global__ void __launch_bounds__(SCATTER_THREADS) permute_scatter_kernel(const int32_t* __restrict__ idx,
                                                                          const float* __restrict__ w, int n, int k,
                                                                          int E, int32_t* __restrict__ offsets,
                                                                          int32_t* __restrict__ row_token,
                                                                          int32_t* __restrict__ row_slot,
                                                                          float* __restrict__ row_w) {
  constexpr int WAVES = SCATTER_THREADS / 64;
  __shared__ int seg_count[WAVES], seg_below[WAVES];
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool dropped = e == E;
  const int seg = ((n + WAVES - 1) / WAVES + 63) & ~63;
  const int s0 = min(n, wave * seg), s1 = min(n, s0 + seg);
  const uint64_t below = (1ull << lane) - 1ull;
  // a block is NB ids per lane, all loaded before any is used; a segment of one block
  // (n <= 16 * 64 * NB) keeps its ids in registers for the second pass
  constexpr int NB = 32;
  int id[NB];
  auto load_block = [&](int b0) {
#pragma unroll
    for (int j = 0; j < NB; ++j) id[j] = idx[min(b0 + 64 * j + lane, n - 1)];   // unconditional, clamped
  };
  auto hit_of = [&](int b0, int j) {
    const int i = b0 + 64 * j + lane;
    const int v = id[j];
    return i < s1 && (dropped ? (v < 0 || v >= E) : v == e);
  };
  // below: routes of experts < e (all valid routes for the dropped workgroup)
  int count = 0, below_e = 0;
  for (int b0 = s0; b0 < s1; b0 += 64 * NB) {
    load_block(b0);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = b0 + 64 * j + lane;
      const int v = id[j];
      count += __popcll(__ballot(hit_of(b0, j)));
      below_e += __popcll(__ballot(i < s1 && v >= 0 && v < e));
    }
  }
  if (lane == 0) {
    seg_count[wave] = count;
    seg_below[wave] = below_e;
  }
  __syncthreads();
  int base = 0;
  for (int q = 0; q < WAVES; ++q) base += seg_below[q];
  if (threadIdx.x == 0) offsets[e] = base;
  int pos = base;
  for (int q = 0; q < wave; ++q) pos += seg_count[q];
  const bool one_block = s1 - s0 <= 64 * NB;
  for (int b0 = s0; b0 < s1; b0 += 64 * NB) {
    if (!one_block) load_block(b0);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = b0 + 64 * j + lane;
      const bool hit = hit_of(b0, j);
      const uint64_t mask = __ballot(hit);
      if (hit) {
        const int p = pos + __popcll(mask & below);
        row_token[p] = i / k;
        row_slot[p] = i - (i / k) * k;
        row_w[p] = dropped ? 0.0f : w[i];
      }
      pos += __popcll(mask);
    }
  }
}

// n <= 1024 routes (batched decode) in one workgroup: permute_small_body
// (permute_small.h), which the batched decode's prep launch also runs.
__global__ void __launch_bounds__(PERMUTE_THREADS) permute_small_kernel(const int32_t* __restrict__ idx,
                                                                        const float* __restrict__ w, int n, int k,
                                                                        int E, int32_t* __restrict__ offsets,
                                                                        int32_t* __restrict__ row_token,
                                                                        int32_t* __restrict__ row_slot,
                                                                        float* __restrict__ row_w) {
  permute_small_body<PERMUTE_THREADS>(idx, w, n, k, E, offsets, row_token, row_slot, row_w);
}

// y rows of the dropped routes (rows [offsets[E], n) of the permutation) are
// zero, so the combine adds nothing for them.  Runs before the expert kernels:
// rows a caller's own permutation left undefined there are overwritten by the
// expert kernels afterwards, and entries outside [0, T) x [0, k) are skipped.
__global__ void __launch_bounds__(256) drop_zero_kernel(const int32_t* __restrict__ offsets, int E, int n, int T,
                                                        int k, int D, const int32_t* __restrict__ row_token,
                                                        const int32_t* __restrict__ row_slot,
                                                        uint16_t* __restrict__ y) {
  const int first = offsets[E];
  const int per_row = D / 8;   // 16-byte stores
  const int64_t total = (int64_t)max(n - first, 0) * per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int r = first + (int)(i / per_row);
    const int c = (int)(i - (int64_t)(r - first) * per_row);
    const int t = row_token[r], sl = row_slot[r];
    if (t < 0 || t >= T || sl < 0 || sl >= k) continue;
    reinterpret_cast<uint4*>(y + ((int64_t)t * k + sl) * D)[c] = uint4{0u, 0u, 0u, 0u};
  }
}

// tiles[t] = (expert, first row of the tile); count in tiles_n[0].
__global__ void __launch_bounds__(1024) tile_list_kernel(const int32_t* __restrict__ offsets, int E, int MT,
                                                         int2* __restrict__ tiles, int32_t* __restrict__ tiles_n,
                                                         uint32_t* __restrict__ zeros) {
  __shared__ int sc[1024];
  if (threadIdx.x < ZERO_WORDS) zeros[threadIdx.x] = 0u;   // source of the zero A columns past K
  // one thread per expert (E <= 1024): its tile count, then an inclusive scan (Hillis-Steele)
  const int e = threadIdx.x;
  int cnt = 0;
  if (e < E) {
    const int rows = offsets[e + 1] - offsets[e];
    cnt = rows > 0 ? 1 + (rows - 1) / MT : 0;
  }
  sc[e] = cnt;
  __syncthreads();
  for (int off = 1; off < 1024; off *= 2) {
    const int v = e >= off ? sc[e - off] : 0;
    __syncthreads();
    sc[e] += v;
    __syncthreads();
  }
  const int first = sc[e] - cnt;
  if (e == 1023) tiles_n[0] = sc[1023];
  for (int t = 0; t < cnt; ++t) tiles[first + t] = make_int2(e, offsets[e] + t * MT);
}

// ------------------------------------------------------------ grouped GEMM ---
struct GroupedArgs {
  const uint16_t* a;            // A source rows (x [T, D] or h [rows, F]), bf16
  int a_stride;                 // elements per A source row
  const int32_t* a_gather;      // A source row of tile row r (row_token) or null (row r itself)
  const uint8_t* pool;
  Layout L;
  const int32_t* slot_table;    // [E] slot of expert e (-1: not resident)
  const int32_t* offsets;       // [E+1]
  const int2* tiles;
  const int32_t* tiles_n;
  const int32_t* row_token;
  const int32_t* row_slot;
  const float* row_w;
  int K, N, k;
  float limit;
  uint16_t* out;                // gate/up: h [rows, N]; down: y [T, k, N]
};

// LDS: A double buffer (MT rows x 272 B), per-row chunk sums (2-bit), then the
// staged scales (2-bit: scales and biases of each matrix; FP4: E8M0 bytes).
// Activation sums per staged row and chunk: one per group (2-bit g128: one).
constexpr int sums_per_row(int kind) { return is_aff(kind) ? KC / aff_group(kind) : 1; }
template <int KIND, int MT>
struct GroupedLds {
  static constexpr int A = 2 * MT * A_ROW_BYTES;
  static constexpr int SUMS = 2 * MT * sums_per_row(KIND) * 4;
};
inline size_t grouped_lds_bytes(int kind, int MT, int NM, int K) {
  const bool affine = kind == KIND_Q2 || is_aff(kind);
  const int g = kind == KIND_Q2 ? KC : (is_aff(kind) ? aff_group(kind) : 32);
  const int per_row = (K + g - 1) / g;
  const size_t scales = affine ? (size_t)2 * NM * NT * per_row * 2 : (size_t)NM * NT * per_row;
  return (size_t)2 * MT * A_ROW_BYTES + (size_t)2 * MT * sums_per_row(kind) * 4 + scales;
}

// Stage chunk c of the tile's A rows: MT rows x 128 values, 16 values per item
// (8 items per row).  2-bit: each 8-value piece in MFMA order, plus the row's
// chunk sum; FP4: natural order.  Rows past the tile's end and columns past K are
// zero.
template <int KIND, int MT>
struct AStage {
  static constexpr int ITEMS = (MT * 8 + 255) / 256;   // per thread (MT * 8 items in all)
  uint4 v[ITEMS][2];

  __device__ __forceinline__ void load(const GroupedArgs& g, int row0, int rows, int c) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int item = threadIdx.x + 256 * i;
      const int r = item >> 3;
      const int col = c * KC + (item & 7) * 16;
      const bool live = item < MT * 8 && r < rows && col < g.K;
      const int src_row = live ? (g.a_gather ? g.a_gather[row0 + r] : row0 + r) : 0;
      const uint4* p = reinterpret_cast<const uint4*>(g.a + (size_t)src_row * g.a_stride + (live ? col : 0));
      v[i][0] = p[0];
      v[i][1] = p[1];
      if (!live) v[i][0] = v[i][1] = make_uint4(0, 0, 0, 0);
    }
  }

  __device__ __forceinline__ void store(uint8_t* abuf, float* sums) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int item = threadIdx.x + 256 * i;
      const int r = item >> 3;
      uint4 lo = v[i][0], hi = v[i][1];
      if constexpr (KIND == KIND_Q2) {
        pairs_mfma(v[i][0].x, v[i][0].y, lo.x, lo.y);
        pairs_mfma(v[i][0].z, v[i][0].w, lo.z, lo.w);
        pairs_mfma(v[i][1].x, v[i][1].y, hi.x, hi.y);
        pairs_mfma(v[i][1].z, v[i][1].w, hi.z, hi.w);
        const float s = sum8_lanes(sum_bf16x8(lo) + sum_bf16x8(hi));
        if (item < MT * 8 && (item & 7) == 0) sums[r] = s;
      } else if constexpr (is_aff(KIND)) {
        // natural order; the sum of each group's G / 16 items (aligned lanes)
        constexpr int P = aff_group(KIND) / 16;
        float s = sum_bf16x8(lo) + sum_bf16x8(hi);
        s = s + __uint_as_float(xor1_u32(__float_as_uint(s)));
        if constexpr (P >= 4) s = s + __uint_as_float(xor2_u32(__float_as_uint(s)));
        if constexpr (P >= 8) s = s + __uint_as_float(mirror8_u32(__float_as_uint(s)));
        if (item < MT * 8 && (item % P) == 0) sums[r * (8 / P) + (item & 7) / P] = s;
      }
      if (item < MT * 8) {
        uint4* d = reinterpret_cast<uint4*>(abuf + r * A_ROW_BYTES + (item & 7) * 32);
        d[0] = lo;
        d[1] = hi;
      }
    }
  }
};

// The lane's codes of chunk c for weight row `row` of one matrix.
// 2-bit: lane group kg owns codes [32kg, 32kg+32) of the group = 8 bytes.
// FP4: lane group kg owns block kg of the chunk = 16 bytes.
// Other affine widths: at step s lane group kg takes codes 32 s + 8 kg .. + 7 of the
// chunk (BITS bytes of the row's bit stream), loaded for all four steps at once.
template <int KIND, bool AFF = is_aff(KIND)>
struct BChunk;

template <int KIND>
struct BChunk<KIND, true> {
  static constexpr int BITS = aff_bits(KIND);
  uint32_t p[4];   // the eight codes of each step, low field first
  __device__ __forceinline__ void load(const uint8_t* wrow, int c, int kg, int row_bytes) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int m = 16 * c + 4 * s + kg;   // piece index: BITS bytes each
      if constexpr (BITS == 2) {
        p[s] = *reinterpret_cast<const uint16_t*>(wrow + min(2 * m, row_bytes - 2));
      } else if constexpr (BITS == 4) {
        p[s] = *reinterpret_cast<const uint32_t*>(wrow + min(4 * m, row_bytes - 4));
      } else {   // 3 bytes at 3 m: the two words around them
        const int bit = 24 * m, wb = (bit >> 5) * 4;
        const uint32_t w0 = *reinterpret_cast<const uint32_t*>(wrow + min(wb, row_bytes - 4));
        const uint32_t w1 = *reinterpret_cast<const uint32_t*>(wrow + min(wb + 4, row_bytes - 4));
        p[s] = __builtin_amdgcn_alignbit(w1, w0, bit & 31) & 0xFFFFFFu;
      }
    }
  }
  // codes 0..15 are exact in bf16 (the float's upper half)
  __device__ __forceinline__ bf16x8_t step(int s, float) const {
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float f0 = (float)((p[s] >> (BITS * 2 * t)) & MASK);
      const float f1 = (float)((p[s] >> (BITS * (2 * t + 1))) & MASK);
      o[t] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
    }
    return __builtin_bit_cast(bf16x8_t, o);
  }
};

template <int KIND>
struct BChunk<KIND, false> {
  uint4 v;
  __device__ __forceinline__ void load(const uint8_t* wrow, int c, int kg, int row_bytes) {
    if constexpr (KIND == KIND_Q2) {
      const int off = min(c * 32 + kg * 8, row_bytes - 8);
      const uint2 t = *reinterpret_cast<const uint2*>(wrow + off);
      v = make_uint4(t.x, t.y, 0, 0);
    } else {
      const int off = min(c * 64 + kg * 16, row_bytes - 16);
      v = *reinterpret_cast<const uint4*>(wrow + off);
    }
  }
  __device__ __forceinline__ bf16x8_t step(int s, float scale) const {
    if constexpr (KIND == KIND_Q2) {
      const uint32_t wd = (s >> 1) ? v.y : v.x;
      return (s & 1) ? q2_codes_to_b<1>(wd) : q2_codes_to_b<0>(wd);
    } else {
      return fp4_codes_to_b(word_of(v, s), scale);
    }
  }
};

// Per-lane accumulation of one K chunk for NM matrices over MT/16 token blocks:
// each step converts the lane's codes once per matrix and feeds every token block.
template <int KIND, int MT, int NM>
__device__ __forceinline__ void chunk_mma(const uint8_t* abuf, const float* sums, const BChunk<KIND> (&b)[NM],
                                          const float (&scale)[NM], const float (&bias)[NM], int lane,
                                          f32x4_t (&acc)[NM][MT / 16]) {
  const int i = lane & 15, kg = lane >> 4;
  f32x4_t c[NM][MT / 16];
  if constexpr (KIND == KIND_Q2) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int tb = 0; tb < MT / 16; ++tb) c[m][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8_t bv[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) bv[m] = b[m].step(s, scale[m]);
#pragma unroll
    for (int tb = 0; tb < MT / 16; ++tb) {
      const bf16x8_t a = lds_a(abuf, (tb * 16 + i) * A_ROW_BYTES + kg * 64 + s * 16);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if constexpr (KIND == KIND_Q2) c[m][tb] = mfma(a, bv[m], c[m][tb]);
        else acc[m][tb] = mfma(a, bv[m], acc[m][tb]);
      }
    }
  }
  if constexpr (KIND == KIND_Q2) {
    // D rows of this lane are tokens tb*16 + 4kg + r: the group formula per token
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int tb = 0; tb < MT / 16; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[m][tb][r] = acc[m][tb][r] + (scale[m] * c[m][tb][r] + bias[m] * sums[tb * 16 + 4 * kg + r]);
  }
}

// Other affine widths: the chunk's 128 / G groups in turn, each G / 32 steps (A read at
// codes 32 s + 8 kg, natural order), the group formula after each group's last step;
// ngroups: the chunk's groups inside the row (the last chunk of a K that is not a whole
// number of chunks holds fewer; the rest see zero activations and are skipped).
template <int KIND, int MT, int NM>
__device__ __forceinline__ void chunk_mma_aff(const uint8_t* abuf, const float* sums, const BChunk<KIND> (&b)[NM],
                                              const float (&scale)[NM][4], const float (&bias)[NM][4], int ngroups,
                                              int lane, f32x4_t (&acc)[NM][MT / 16]) {
  constexpr int SPG = aff_group(KIND) / 32, NGC = KC / aff_group(KIND);
  const int i = lane & 15, kg = lane >> 4;
  f32x4_t c[NM][MT / 16];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int tb = 0; tb < MT / 16; ++tb) c[m][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8_t bv[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) bv[m] = b[m].step(s, 1.0f);
#pragma unroll
    for (int tb = 0; tb < MT / 16; ++tb) {
      const bf16x8_t a = lds_a(abuf, (tb * 16 + i) * A_ROW_BYTES + s * 64 + kg * 16);
#pragma unroll
      for (int m = 0; m < NM; ++m) c[m][tb] = mfma(a, bv[m], c[m][tb]);
    }
    if ((s + 1) % SPG == 0) {
      const int grp = s / SPG;
      if (grp < ngroups) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int tb = 0; tb < MT / 16; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[m][tb][r] = acc[m][tb][r] +
                              (scale[m][grp] * c[m][tb][r] + bias[m][grp] * sums[(tb * 16 + 4 * kg + r) * NGC + grp]);
      }
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int tb = 0; tb < MT / 16; ++tb) c[m][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
}

// Scale of (row j of the workgroup, chunk c) for tensor q: 2-bit bf16 scale/bias of
// group c; FP4 E8M0 of block 4c + kg.
template <int KIND>
__device__ __forceinline__ float staged_scale(const uint8_t* sc, int q, int j, int c, int kg, int per_row, bool f16) {
  if constexpr (KIND == KIND_Q2 || is_aff(KIND)) {   // c: the group
    return scale_bits_to_f32(reinterpret_cast<const uint16_t*>(sc)[(q * NT + j) * per_row + c], f16);
  } else {
    // blocks past K (the last chunk of K = 2880) meet zero activations: any finite scale
    return 4 * c + kg < per_row ? e8m0_to_f32(sc[(q * NT + j) * per_row + 4 * c + kg]) : 1.0f;
  }
}

// Shared main loop of both grouped kernels.  NM = 2 (W1, W3) or 1 (W2); tq =
// kernel tensor indices of the matrices (codes) in the record layout.
template <int KIND, int MT, int NM>
__device__ __forceinline__ bool grouped_main(const GroupedArgs& g, uint8_t* lds, const int (&tq)[NM], int& e,
                                             int& row0, int& rows, f32x4_t (&acc)[NM][MT / 16]) {
  using Lds = GroupedLds<KIND, MT>;
  constexpr bool AQ = KIND == KIND_Q2 || is_aff(KIND);   // affine: scales and biases per group
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kg = lane >> 4;
  if ((int)blockIdx.x >= g.tiles_n[0]) return false;
  const int2 tile = g.tiles[blockIdx.x];
  e = tile.x;
  row0 = tile.y;
  rows = min(MT, g.offsets[e + 1] - row0);
  const int n0 = blockIdx.y * NT;
  const int slot = g.slot_table[e];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int tb = 0; tb < MT / 16; ++tb) acc[m][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (slot < 0) return true;   // not resident: zero rows

  uint8_t* abuf[2] = {lds, lds + MT * A_ROW_BYTES};
  float* sums[2] = {reinterpret_cast<float*>(lds + Lds::A),
                    reinterpret_cast<float*>(lds + Lds::A) + MT * sums_per_row(KIND)};
  uint8_t* sc = lds + Lds::A + Lds::SUMS;
  const uint8_t* base = g.pool + (int64_t)slot * g.L.record_bytes;
  const int nchunks = (g.K + KC - 1) / KC;
  // bytes per weight row and per scale row
  constexpr int GRP = is_aff(KIND) ? aff_group(KIND) : KC;
  const int groups = (g.K + GRP - 1) / GRP;                     // affine: stored groups per row
  const int row_bytes = KIND == KIND_Q2 ? groups * 32 : (is_aff(KIND) ? groups * GRP * aff_bits(KIND) / 8 : g.K / 2);
  const int per_row = AQ ? groups : g.K / 32;                   // scale entries per row
  const int row = n0 + wave * 16 + (lane & 15);
  const uint8_t* wrow[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) wrow[m] = base + g.L.off[tq[m]] + (int64_t)row * row_bytes;

  // scales (and biases) of the 64 weight rows: contiguous runs, straight into LDS
  {
    const int run = NT * per_row * (AQ ? 2 : 1);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      // 2-bit: slot 2m = scales, 2m+1 = biases; FP4: slot m = E8M0 bytes
      const int q = AQ ? 2 * m : m;
      dma_to_lds(base + g.L.off[tq[m] + 1] + (int64_t)n0 * run / NT, sc + q * run, run, (wave + m) & 3, 4, lane);
      if constexpr (AQ)
        dma_to_lds(base + g.L.off[tq[m] + 2] + (int64_t)n0 * run / NT, sc + (q + 1) * run, run, (wave + m + 2) & 3,
                   4, lane);
    }
  }
  AStage<KIND, MT> as;
  BChunk<KIND> bc[NM], bn[NM];
  as.load(g, row0, rows, 0);
#pragma unroll
  for (int m = 0; m < NM; ++m) bc[m].load(wrow[m], 0, kg, row_bytes);
  as.store(abuf[0], sums[0]);
  wait_vmem();
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int cur = c & 1;
    const bool more = c + 1 < nchunks;
    if (more) {
      as.load(g, row0, rows, c + 1);
#pragma unroll
      for (int m = 0; m < NM; ++m) bn[m].load(wrow[m], c + 1, kg, row_bytes);
    }
    if constexpr (is_aff(KIND)) {
      constexpr int NGC = KC / GRP;
      const int g0 = c * NGC, ng = min(NGC, groups - g0);
      float scale[NM][4], bias[NM][4];
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int q = 0; q < NGC; ++q) {
          const int gi = min(g0 + q, groups - 1);
          scale[m][q] = staged_scale<KIND>(sc, 2 * m, wave * 16 + (lane & 15), gi, kg, per_row, g.L.f16);
          bias[m][q] = staged_scale<KIND>(sc, 2 * m + 1, wave * 16 + (lane & 15), gi, kg, per_row, g.L.f16);
        }
      chunk_mma_aff<KIND, MT, NM>(abuf[cur], sums[cur], bc, scale, bias, ng, lane, acc);
    } else {
      float scale[NM], bias[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        // 2-bit: tensor slots 2m (scales) and 2m+1 (biases); FP4: slot 2m (E8M0)
        scale[m] = staged_scale<KIND>(sc, KIND == KIND_Q2 ? 2 * m : m, wave * 16 + (lane & 15), c, kg, per_row, g.L.f16);
        bias[m] = KIND == KIND_Q2 ? staged_scale<KIND>(sc, 2 * m + 1, wave * 16 + (lane & 15), c, kg, per_row, g.L.f16) : 0.0f;
      }
      chunk_mma<KIND, MT, NM>(abuf[cur], sums[cur], bc, scale, bias, lane, acc);
    }
    if (more) {
      as.store(abuf[cur ^ 1], sums[cur ^ 1]);
#pragma unroll
      for (int m = 0; m < NM; ++m) bc[m] = bn[m];
    }
    __syncthreads();
  }
  return true;
}

template <int KIND, int MT>
__global__ void __launch_bounds__(256) grouped_gate_up_kernel(GroupedArgs g) {
  extern __shared__ __align__(16) uint8_t lds[];
  f32x4_t acc[2][MT / 16];
  int e, row0, rows;
  const int tq[2] = {0, 6};   // w1, w3
  if (!grouped_main<KIND, MT, 2>(g, lds, tq, e, row0, rows, acc)) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = blockIdx.y * NT + wave * 16 + (lane & 15);
  const int kg = lane >> 4;
#pragma unroll
  for (int tb = 0; tb < MT / 16; ++tb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tr = tb * 16 + 4 * kg + r;
      if (tr < rows) {
        float gv = round_bf16(acc[0][tb][r]);
        float uv = round_bf16(acc[1][tb][r]);
        if (g.limit > 0.0f) {
          uv = fminf(fmaxf(uv, -g.limit), g.limit);
          gv = fminf(gv, g.limit);
        }
        const float h = (silu_f32(gv) * uv) * g.row_w[row0 + tr];
        g.out[(size_t)(row0 + tr) * g.N + n] = f32_to_bf16(h);
      }
    }
}

template <int KIND, int MT>
__global__ void __launch_bounds__(256) grouped_down_kernel(GroupedArgs g) {
  extern __shared__ __align__(16) uint8_t lds[];
  f32x4_t acc[1][MT / 16];
  int e, row0, rows;
  const int tq[1] = {3};      // w2
  if (!grouped_main<KIND, MT, 1>(g, lds, tq, e, row0, rows, acc)) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = blockIdx.y * NT + wave * 16 + (lane & 15);
  const int kg = lane >> 4;
#pragma unroll
  for (int tb = 0; tb < MT / 16; ++tb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tr = tb * 16 + 4 * kg + r;
      if (tr < rows) {
        const int rr = row0 + tr;
        g.out[((size_t)g.row_token[rr] * g.k + g.row_slot[rr]) * g.N + n] = f32_to_bf16(acc[0][tb][r]);
      }
    }
}

// -------------------------------------------------- FP4 grouped GEMM, large tiles ---
// One 512-thread workgroup = one M tile (128 rows of one expert) x 256 weight rows of
// each matrix (W1 and W3 for gate/up, W2 for down); wave w owns weight rows
// [32w, 32w + 32) as two 16-row fragments and all eight 16-row token fragments.
// The A tile is read once per 256 weight rows (the 64-row tiles read it once per 64)
// and each expert's weights once per 128 of its rows.
// K runs in chunks of 128 through a three-stage LDS ring filled by untracked
// direct-to-LDS loads (one 16-byte slot per lane, gathered rows, rows swizzled by
// XOR so the MFMA reads hit distinct bank groups); each wave's codes and E8M0 scales
// are prefetched two chunks ahead in registers.  Same arithmetic as the 64-row
// kernels: B = E2M1 x 2^e converted exactly to bf16, v_mfma_f32_16x16x32_bf16, fp32.
constexpr int G2_THREADS = 512;
constexpr int G2_WAVES = G2_THREADS / 64;
constexpr int G2_MT = 128;                 // token rows per workgroup (8 fragments)
constexpr int G2_TB = G2_MT / 16;
constexpr int G2_NT = 32 * G2_WAVES;       // 256 weight rows per matrix
constexpr int G2_STAGES = 3;
constexpr int G2_GROUP = 1;                // M tiles per XCD block (workgroup order; 2 measured no faster)
constexpr int G2_ABYTES = G2_MT * 256;     // one A chunk: 128 rows x 128 bf16
constexpr int G2_ASLICES = G2_ABYTES / 1024 / G2_WAVES;   // 1 KiB direct-to-LDS slices per wave and chunk

// Wait until the load that produced v has landed (the compiler's own wait; loads
// complete in issue order, so everything this wave issued before it has too), then
// an LDS-only workgroup barrier.
__device__ __forceinline__ void lds_sync_after(uint32_t v) {
  asm volatile("" ::"v"(v) : "memory");
  lds_sync();
}

// Byte offset of (row r, 16-byte column slot k16) in a staged A chunk.
__device__ __forceinline__ uint32_t g2_aoff(int r, int k16) { return (uint32_t)(r * 256 + ((k16 ^ (r & 15)) << 4)); }

template <int NM>
struct G2Chunk {
  uint4 codes[NM][2];
  uint32_t sc[NM][2];    // raw E8M0 bytes as loaded (a block past K: any byte)
  bool in_k;             // the lane's block of this chunk lies inside K
};

template <int NM>
__device__ __forceinline__ void g2_issue(const GroupedArgs& g, uint8_t* stage, const uint8_t* (&arow)[G2_ASLICES],
                                         const int (&ak16)[G2_ASLICES], const uint8_t* zeros,
                                         const uint8_t* (&wrow)[NM][2],
                                         const uint8_t* (&srow)[NM][2], int c, int kg, int wave, int lane,
                                         int row_bytes, int blocks, G2Chunk<NM>& out) {
  out.in_k = 4 * c + kg < blocks;
  // A: this wave's 1 KiB slices of the chunk (slot = 64 * (G2_ASLICES wave + q) + lane)
#pragma unroll
  for (int q = 0; q < G2_ASLICES; ++q) {
    const int kcol = c * 128 + ak16[q] * 8;
    const uint8_t* src = kcol < g.K ? arow[q] + c * 256 + ak16[q] * 16 : zeros;
    tile::lds_load16_untracked(src, stage + (G2_ASLICES * wave + q) * 1024);
  }
  // B: the lane's 32 codes (block kg of the chunk) and their E8M0 scale, per matrix and fragment
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      out.codes[m][f] = *reinterpret_cast<const uint4*>(wrow[m][f] + min(c * 64 + kg * 16, row_bytes - 16));
      // unconditional (clamped) load: the compiler then counts this wave's loads exactly;
      // the value is checked where it is used, so nothing here waits for it
      out.sc[m][f] = srow[m][f][min(4 * c + kg, blocks - 1)];
    }
}

// ntb: token fragments holding rows of the tile (the rest are skipped, uniformly).
template <int NM>
__device__ __forceinline__ void g2_compute(const uint8_t* ab, const G2Chunk<NM>& ch, int i, int kg, int ntb,
                                           f32x4_t (&acc)[NM][2][G2_TB]) {
  // blocks past K meet zero activations: any finite scale (raw 127 = 1.0)
  float scale[NM][2];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < 2; ++f) scale[m][f] = e8m0_to_f32(ch.in_k ? ch.sc[m][f] : 127u);
  if constexpr (NM == 1) {
    // A fragments in pairs, double-buffered: the next pair's LDS reads are in flight
    // while the current pair's MFMAs run (the next pair of the same step, or the first
    // of the next step); pairs past the tile's rows are skipped (ntb uniform).  (Gate/up
    // has no registers to spare for the second buffer.)
    bf16x8_t cur0 = lds_a(ab, g2_aoff(i, 4 * kg)), cur1 = lds_a(ab, g2_aoff(16 + i, 4 * kg));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8_t bv[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) bv[f] = fp4_codes_to_b(word_of(ch.codes[0][f], s), scale[0][f]);
#pragma unroll
      for (int tp = 0; tp < G2_TB; tp += 2) {
        if (tp >= ntb) break;
        const bool last = tp + 2 >= ntb;
        const int nt = last ? 0 : tp + 2;
        const int ns = last ? min(s + 1, 3) : s;   // after the last step: a read nobody uses
        const bf16x8_t nx0 = lds_a(ab, g2_aoff(nt * 16 + i, 4 * kg + ns));
        const bf16x8_t nx1 = lds_a(ab, g2_aoff((nt + 1) * 16 + i, 4 * kg + ns));
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          acc[0][f][tp] = mfma(cur0, bv[f], acc[0][f][tp]);
          acc[0][f][tp + 1] = mfma(cur1, bv[f], acc[0][f][tp + 1]);
        }
        cur0 = nx0;
        cur1 = nx1;
      }
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8_t bv[NM][2];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < 2; ++f) bv[m][f] = fp4_codes_to_b(word_of(ch.codes[m][f], s), scale[m][f]);
    // token fragments in pairs: both A reads issue before the pair's MFMAs (one LDS
    // round trip per 4 NM MFMAs); a fragment past the tile's rows is computed on
    // stale rows and discarded
#pragma unroll
    for (int tp = 0; tp < G2_TB; tp += 2) {
      if (tp >= ntb) break;
      const bf16x8_t a0 = lds_a(ab, g2_aoff(tp * 16 + i, 4 * kg + s));
      const bf16x8_t a1 = lds_a(ab, g2_aoff((tp + 1) * 16 + i, 4 * kg + s));
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          acc[m][f][tp] = mfma(a0, bv[m][f], acc[m][f][tp]);
          acc[m][f][tp + 1] = mfma(a1, bv[m][f], acc[m][f][tp + 1]);
        }
    }
  }
}

// grid = slices * tiles rounded up to 8 G2_GROUP, one dimension, slices = ceil(N / 256).
// Workgroups are dealt to the eight XCDs round-robin by launch index (b % 8).  XCD x takes
// blocks of G2_GROUP consecutive tiles (block j of XCD x: tiles (8 j + x) G2_GROUP ..) and
// runs a block's workgroups slice by slice, its tiles inside a slice, so the slices of an
// M tile run on one XCD together and its gathered A rows are fetched into that XCD's L2
// once instead of once per XCD (G2_GROUP > 1 would also share weight slices between a
// block's tiles).  NM = 2: gate/up (W1, W3) -> h; NM = 1: down (W2) -> y.
template <int NM>
__global__ void __launch_bounds__(G2_THREADS) g2_fp4_kernel(GroupedArgs g, const uint8_t* __restrict__ zeros,
                                                            int slices) {
  __shared__ __align__(16) uint8_t abuf[G2_STAGES][G2_ABYTES];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, kg = lane >> 4;
  const int b8 = blockIdx.x >> 3;                         // sequence number on this XCD
  const int blk = b8 / (slices * G2_GROUP), w = b8 - blk * (slices * G2_GROUP);
  const int slice = w / G2_GROUP;
  const int tile_id = (blk * 8 + (int)(blockIdx.x & 7)) * G2_GROUP + (w - slice * G2_GROUP);
  if (tile_id >= g.tiles_n[0]) return;
  const int2 tl = g.tiles[tile_id];
  const int e = tl.x, row0 = tl.y;
  const int rows = min(G2_MT, g.offsets[e + 1] - row0);
  const int ntb = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
  const int slot = g.slot_table[e];
  f32x4_t acc[NM][2][G2_TB];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int tb = 0; tb < G2_TB; ++tb) acc[m][f][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int nw0 = slice * G2_NT + 32 * wave;   // the wave's first weight row
  if (slot >= 0) {
    const int nch = (g.K + 127) / 128;
    const int row_bytes = g.K / 2, blocks = g.K / 32;
    // A sources of the lane's two slots per chunk
    const uint8_t* arow[G2_ASLICES];
    int ak16[G2_ASLICES];
#pragma unroll
    for (int q = 0; q < G2_ASLICES; ++q) {
      const int S = 64 * (G2_ASLICES * wave + q) + lane;
      const int r = S >> 4;
      ak16[q] = (S & 15) ^ (r & 15);
      const int rr = min(r, rows - 1);   // rows past the tile's end: any valid row (discarded)
      const int src = g.a_gather ? g.a_gather[row0 + rr] : row0 + rr;
      arow[q] = reinterpret_cast<const uint8_t*>(g.a + (size_t)src * g.a_stride);
    }
    const uint8_t* base = g.pool + (int64_t)slot * g.L.record_bytes;
    const int tq[2] = {NM == 2 ? 0 : 3, 6};   // w1, w3 (gate/up) or w2 (down)
    const uint8_t* wrow[NM][2];
    const uint8_t* srow[NM][2];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int n = min(nw0 + 16 * f + i, g.N - 1);   // rows past N: clamped (discarded)
        wrow[m][f] = base + g.L.off[tq[m]] + (int64_t)n * row_bytes;
        srow[m][f] = base + g.L.off[tq[m] + 1] + (int64_t)n * blocks;
      }
    G2Chunk<NM> ring[G2_STAGES];
    // Every issue is unconditional (a chunk past the end re-reads the last one into a
    // stage nothing reads again), so each wait below is for exactly the loads it needs
    // and two chunks stay in flight; a load under a branch makes the compiler wait for all.
    g2_issue<NM>(g, abuf[0], arow, ak16, zeros, wrow, srow, 0, kg, wave, lane, row_bytes, blocks, ring[0]);
    g2_issue<NM>(g, abuf[1], arow, ak16, zeros, wrow, srow, min(1, nch - 1), kg, wave, lane, row_bytes, blocks,
                 ring[1]);
    // three chunks per trip so every ring index is a compile-time constant
    for (int c0 = 0; c0 < nch; c0 += G2_STAGES) {
#pragma unroll
      for (int u = 0; u < G2_STAGES; ++u) {
        const int c = c0 + u;
        // this wave's loads of chunk c have landed (its codes are consumed here, and
        // its earlier direct-to-LDS loads complete first); then every wave's
        lds_sync_after(ring[u].codes[NM - 1][1].w);
        // into the stage chunk c - 1 used: every wave is past it
        g2_issue<NM>(g, abuf[(u + 2) % G2_STAGES], arow, ak16, zeros, wrow, srow, min(c + 2, nch - 1), kg, wave,
                     lane, row_bytes, blocks, ring[(u + 2) % G2_STAGES]);
        if (c < nch) g2_compute<NM>(abuf[u], ring[u], i, kg, ntb, acc);
      }
    }
    // the re-reads issued past the end (direct-to-LDS among them) land before the
    // workgroup's LDS is released
    tile::wait_vmem();
  }
  // epilogue: lane holds rows tb*16 + 4kg + r (tokens) x column nw0 + 16f + i
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int n = nw0 + 16 * f + i;
    if (n >= g.N) continue;
#pragma unroll
    for (int tb = 0; tb < G2_TB; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tr = tb * 16 + 4 * kg + r;
        if (tr >= rows) continue;
        const int rr = row0 + tr;
        if constexpr (NM == 2) {
          float gv = round_bf16(acc[0][f][tb][r]);
          float uv = round_bf16(acc[1][f][tb][r]);
          if (g.limit > 0.0f) {
            uv = fminf(fmaxf(uv, -g.limit), g.limit);
            gv = fminf(gv, g.limit);
          }
          g.out[(size_t)rr * g.N + n] = f32_to_bf16((silu_f32(gv) * uv) * g.row_w[rr]);
        } else {
          g.out[((size_t)g.row_token[rr] * g.k + g.row_slot[rr]) * g.N + n] = f32_to_bf16(acc[0][f][tb][r]);
        }
      }
  }
}

// out[t, d] = bf16(0 + y[t,0,d] + ... + y[t,k-1,d] (+ addend[t,d])); routed likewise in fp32.
__global__ void __launch_bounds__(256) combine_kernel(const uint16_t* __restrict__ y, const uint16_t* __restrict__ addend,
                                                      int T, int k, int D, float* __restrict__ routed,
                                                      uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // one pair of columns
  const int64_t pairs = (int64_t)T * D / 2;
  if (i >= pairs) return;
  const int64_t t = (2 * i) / D;
  const int d = (int)(2 * i - t * D);
  float a0 = 0.0f, a1 = 0.0f;
  for (int s = 0; s < k; ++s) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(y + ((size_t)t * k + s) * D + d);
    a0 = a0 + bf16_to_f32((uint16_t)(v & 0xffff));
    a1 = a1 + bf16_to_f32((uint16_t)(v >> 16));
  }
  if (routed) {
    routed[t * D + d] = a0;
    routed[t * D + d + 1] = a1;
  }
  if (out) {
    float o0 = a0, o1 = a1;
    if (addend) {
      const uint32_t av = *reinterpret_cast<const uint32_t*>(addend + t * D + d);
      o0 = o0 + bf16_to_f32((uint16_t)(av & 0xffff));
      o1 = o1 + bf16_to_f32((uint16_t)(av >> 16));
    }
    *reinterpret_cast<uint32_t*>(out + t * D + d) = (uint32_t)f32_to_bf16(o0) | ((uint32_t)f32_to_bf16(o1) << 16);
  }
}

// The same, 8 columns per thread with 16-byte loads and stores (D a multiple of 8,
// 16-byte aligned arrays): the k slot loads of a thread are all in flight together,
// and each column is summed in the same order as above.
__global__ void __launch_bounds__(256) combine8_kernel(const uint16_t* __restrict__ y,
                                                       const uint16_t* __restrict__ addend, int T, int k, int D,
                                                       float* __restrict__ routed, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // one group of 8 columns
  const int64_t groups = (int64_t)T * D / 8;
  if (i >= groups) return;
  const int64_t t = (8 * i) / D;
  const int d = (int)(8 * i - t * D);
  uint4 v[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
    if (s < k) v[s] = *reinterpret_cast<const uint4*>(y + ((size_t)t * k + s) * D + d);
  float a[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) a[c] = 0.0f;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s >= k) break;
    const uint32_t w[4] = {v[s].x, v[s].y, v[s].z, v[s].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[2 * q] = a[2 * q] + bf16_to_f32((uint16_t)(w[q] & 0xffff));
      a[2 * q + 1] = a[2 * q + 1] + bf16_to_f32((uint16_t)(w[q] >> 16));
    }
  }
  if (routed) {
    float4* r = reinterpret_cast<float4*>(routed + t * D + d);
    r[0] = make_float4(a[0], a[1], a[2], a[3]);
    r[1] = make_float4(a[4], a[5], a[6], a[7]);
  }
  if (out) {
    if (addend) {
      const uint4 av = *reinterpret_cast<const uint4*>(addend + t * D + d);
      const uint32_t w[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[2 * q] = a[2 * q] + bf16_to_f32((uint16_t)(w[q] & 0xffff));
        a[2 * q + 1] = a[2 * q + 1] + bf16_to_f32((uint16_t)(w[q] >> 16));
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = (uint32_t)f32_to_bf16(a[2 * q]) | ((uint32_t)f32_to_bf16(a[2 * q + 1]) << 16);
    *reinterpret_cast<uint4*>(out + t * D + d) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Workspace of a grouped call: [tiles_n][tiles][hidden][x planes], 256-byte aligned regions.
// hidden: rows x F bf16, or rows x ceil(F / 128) plane blocks (matrix-core batched decode);
// x planes: T x D / 128 plane blocks (same).
struct GroupedWs {
  size_t tiles_n, tiles, hidden, xplanes, mx, total;
  int max_tiles;
};

inline GroupedWs grouped_ws(int T, int k, int E, int D, int F) {
  GroupedWs w;
  const int rows = T * k;
  w.max_tiles = rows / 16 + std::min(E, rows) + 1;   // bound for MT >= 16
  w.tiles_n = 0;
  w.tiles = 256;
  // int2 tiles, or one int4 record per active expert (matrix-core batched decode)
  w.hidden = w.tiles + align256(std::max((size_t)w.max_tiles * sizeof(int2), (size_t)std::min(E, rows) * sizeof(int4)));
  const size_t hid = std::max((size_t)rows * F * sizeof(uint16_t), (size_t)rows * ((F + 127) / 128) * 320);
  w.xplanes = w.hidden + align256(hid);
  w.mx = w.xplanes + align256((size_t)T * ((D + 127) / 128) * 320);
  w.total = w.mx + (k > 0 && D > 0 ? prefill_mx_ws_bytes(T, k, D, F) : 0);
  return w;
}


template <int KIND, int MT>
int launch_grouped_mt(const GroupedArgs& gu, const GroupedArgs& dn, int max_tiles, size_t lds_gu, size_t lds_dn,
                      hipStream_t s) {
  auto kgu = grouped_gate_up_kernel<KIND, MT>;
  auto kdn = grouped_down_kernel<KIND, MT>;
  if (lds_gu > 65536 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kgu), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_gu) != hipSuccess)
    return fail(CACHALOT_EHIP, "grouped experts: cannot grant %zu bytes of LDS", lds_gu);
  if (lds_dn > 65536 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kdn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_dn) != hipSuccess)
    return fail(CACHALOT_EHIP, "grouped experts: cannot grant %zu bytes of LDS", lds_dn);
  hipLaunchKernelGGL(kgu, dim3(max_tiles, gu.N / NT), dim3(256), lds_gu, s, gu);
  int rc = check_launch("grouped_gate_up_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(kdn, dim3(max_tiles, dn.N / NT), dim3(256), lds_dn, s, dn);
  return check_launch("grouped_down_kernel");
}

// The earlier kernels stay selectable (CACHALOT_GROUPED_SMALL=1) for comparison: 64-row
// tiles for FP4 prefill, bf16 MFMA for 2-bit batched decode.
inline bool small_tiles_requested() {
  const char* env = getenv("CACHALOT_GROUPED_SMALL");
  return env && env[0] == '1';
}

// FP4 and 2-bit g128 prefill run on the block-scaled matrix cores (prefill_mx.hip)
// unless CACHALOT_PREFILL_BF16=1 selects the bf16-MFMA kernels (g2_fp4_kernel, the
// 64-row grouped kernels).
inline bool prefill_bf16_requested() {
  const char* env = getenv("CACHALOT_PREFILL_BF16");
  return env && env[0] == '1';
}

template <int KIND>
int launch_grouped(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                   const int32_t* slot_table, const int32_t* offsets, const int32_t* row_token,
                   const int32_t* row_slot, const float* row_w, int T, int D, int F, int E, int k, float limit,
                   uint16_t* y, void* workspace, size_t workspace_bytes, hipStream_t s, const char* who,
                   const int32_t* ridx = nullptr, const float* rw = nullptr) {
  // ridx / rw: the routes [T, k], permuted here into offsets / row_* (outputs then)
  CACHALOT_REQUIRE(x && pool && layout && slot_table && offsets && row_token && row_slot && row_w && y,
                   "%s: null pointer", who);
  CACHALOT_REQUIRE((ridx == nullptr) == (rw == nullptr), "%s: routes need both ids and weights", who);
  CACHALOT_REQUIRE(T >= 1, "%s: x must contain at least one token (T=%d)", who, T);
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "%s: k=%d outside 1..%d", who, k, KMAX);
  CACHALOT_REQUIRE(E >= 1 && E <= 1024, "%s: E=%d outside 1..1024", who, E);
  CACHALOT_REQUIRE(D % NT == 0 && D >= 128 && D <= KC * MAX_GROUPS,
                   "%s: D=%d must be a multiple of 64 in 128..8192", who, D);
  CACHALOT_REQUIRE(F % NT == 0 && F >= 64 && F <= KC * MAX_GROUPS, "%s: F=%d must be a multiple of 64 in 64..8192",
                   who, F);
  if (KIND == KIND_Q2 || is_aff(KIND))
    CACHALOT_REQUIRE(D % KC == 0, "%s: D=%d must be a multiple of the 128-code chunk", who, D);
  const GroupedWs wo = grouped_ws(T, k, E, D, F);
  if (workspace == nullptr || workspace_bytes < wo.total)
    return fail(CACHALOT_ESPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, wo.total);
  Layout L;
  static const int used_q2[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  static const int used_fp4[6] = {0, 1, 3, 4, 6, 7};
  int rc = KIND == KIND_Q2 || is_aff(KIND) ? make_layout(layout, 9, used_q2, L, who)
                                           : make_layout(layout, 6, used_fp4, L, who);
  if (rc) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* tiles_n = reinterpret_cast<int32_t*>(ws + wo.tiles_n);
  int2* tiles = reinterpret_cast<int2*>(ws + wo.tiles);
  uint16_t* hidden = reinterpret_cast<uint16_t*>(ws + wo.hidden);
  // tiles of 64 rows when experts see many tokens, 16 for batched decode
  const int MT = T * k >= 4 * E ? 64 : 16;
  uint32_t* zeros = reinterpret_cast<uint32_t*>(ws + wo.tiles_n + 128);
  const bool batched = KIND == KIND_Q2 && MT == 16 && q2mx_supported(D, F, k) && !small_tiles_requested();
  // routes given: permuted by the batched prep launch when one workgroup holds them, else here
  const bool fused = ridx != nullptr && batched && T * k <= PERMUTE_THREADS;
  if (ridx != nullptr && !fused) {
    rc = cachalot_permute(ridx, rw, T, k, E, const_cast<int32_t*>(offsets), const_cast<int32_t*>(row_token),
                          const_cast<int32_t*>(row_slot), const_cast<float*>(row_w), s);
    if (rc) return rc;
  }
  if (batched) {
    // few rows per expert: the matrix-core batched decode, one entry per active expert
    // (its prep launch also clears the dropped routes' y rows)
    return launch_q2mx_batched(x, T, pool, L, slot_table, offsets, E, reinterpret_cast<int4*>(ws + wo.tiles),
                               tiles_n, std::min(E, T * k), row_token, row_slot, row_w, D, F, k, limit,
                               ws + wo.hidden, ws + wo.xplanes, y, s, fused ? ridx : nullptr, fused ? rw : nullptr);
  }
  hipLaunchKernelGGL(drop_zero_kernel, dim3(16), dim3(256), 0, s, offsets, E, T * k, T, k, D, row_token, row_slot, y);
  rc = check_launch("drop_zero_kernel");
  if (rc) return rc;
  const int max_tiles = (T * k) / MT + std::min(E, T * k) + 1;
  if (KIND == KIND_FP4 && MT == 64 && prefill_mx_supported(D, F, L) && !small_tiles_requested() &&
      !prefill_bf16_requested() && max_tiles <= (1 << 20)) {
    hipLaunchKernelGGL(tile_list_kernel, dim3(1), dim3(1024), 0, s, offsets, E, prefill_mx_mt(), tiles, tiles_n, zeros);
    rc = check_launch("tile_list_kernel");
    if (rc) return rc;
    return launch_prefill_mx(x, T, pool, L, slot_table, offsets, tiles, tiles_n, max_tiles, row_token, row_slot,
                             row_w, D, F, k, limit, ws + wo.mx, y, s);
  }
  if (KIND == KIND_Q2 && MT == 64 && prefill_mx_q2_supported(D, F, L) && !small_tiles_requested() &&
      !prefill_bf16_requested() && max_tiles <= (1 << 20)) {
    // 2-bit g128 prefill on the block-scaled matrix cores (prefill_mx.hip)
    hipLaunchKernelGGL(tile_list_kernel, dim3(1), dim3(1024), 0, s, offsets, E, prefill_mx_mt(), tiles, tiles_n, zeros);
    rc = check_launch("tile_list_kernel");
    if (rc) return rc;
    return launch_prefill_mx_q2(x, T, pool, L, slot_table, offsets, tiles, tiles_n, max_tiles, row_token, row_slot,
                                row_w, D, F, k, limit, ws + wo.mx, y, s);
  }
  if (is_aff(KIND) && MT == 64 && prefill_mx_aff_supported(aff_bits(KIND), aff_group(KIND), D, F, L) &&
      !small_tiles_requested() && !prefill_bf16_requested() && max_tiles <= (1 << 20)) {
    // 2-bit g64, 3- and 4-bit g64 / g128 prefill on the block-scaled matrix cores
    hipLaunchKernelGGL(tile_list_kernel, dim3(1), dim3(1024), 0, s, offsets, E, prefill_mx_mt(), tiles, tiles_n, zeros);
    rc = check_launch("tile_list_kernel");
    if (rc) return rc;
    return launch_prefill_mx_aff(aff_bits(KIND), aff_group(KIND), x, T, pool, L, slot_table, offsets, tiles, tiles_n,
                                 max_tiles, row_token, row_slot, row_w, D, F, k, limit, ws + wo.mx, y, s);
  }
  const bool large = KIND == KIND_FP4 && MT == 64 && D % 128 == 0 && F % 32 == 0 && !small_tiles_requested() &&
                     max_tiles <= (1 << 20);
  hipLaunchKernelGGL(tile_list_kernel, dim3(1), dim3(1024), 0, s, offsets, E, large ? G2_MT : MT, tiles, tiles_n,
                     zeros);
  rc = check_launch("tile_list_kernel");
  if (rc) return rc;
  GroupedArgs gu{x, D, row_token, pool, L, slot_table, offsets, tiles, tiles_n, row_token, row_slot, row_w,
                 D, F, k, limit, hidden};
  GroupedArgs dn{hidden, F, nullptr, pool, L, slot_table, offsets, tiles, tiles_n, row_token, row_slot, row_w,
                 F, D, k, limit, y};
  if (large) {
    const int tiles8 = (max_tiles + 8 * G2_GROUP - 1) / (8 * G2_GROUP) * (8 * G2_GROUP);
    const int s_gu = (F + G2_NT - 1) / G2_NT, s_dn = (D + G2_NT - 1) / G2_NT;
    hipLaunchKernelGGL(g2_fp4_kernel<2>, dim3(s_gu * tiles8), dim3(G2_THREADS), 0, s, gu,
                       reinterpret_cast<const uint8_t*>(zeros), s_gu);
    rc = check_launch("g2_fp4_kernel<2>");
    if (rc) return rc;
    hipLaunchKernelGGL(g2_fp4_kernel<1>, dim3(s_dn * tiles8), dim3(G2_THREADS), 0, s, dn,
                       reinterpret_cast<const uint8_t*>(zeros), s_dn);
    return check_launch("g2_fp4_kernel<1>");
  }
  const size_t lds_gu = grouped_lds_bytes(KIND, MT, 2, D), lds_dn = grouped_lds_bytes(KIND, MT, 1, F);
  return MT == 64 ? launch_grouped_mt<KIND, 64>(gu, dn, max_tiles, lds_gu, lds_dn, s)
                  : launch_grouped_mt<KIND, 16>(gu, dn, max_tiles, lds_gu, lds_dn, s);
}

}  // namespace

// The other affine widths on the bf16-MFMA grouped kernels (called by
// cachalot_grouped_experts_affine, affine.hip): workspace and launch.
size_t grouped_affine_ws_bytes(int T, int k, int E, int D, int F) { return grouped_ws(T, k, E, D, F).total; }

int launch_grouped_affine(int bits, int group, const uint16_t* x, const uint8_t* pool,
                          const cachalot_expert_layout* layout, const int32_t* slot_table, const int32_t* offsets,
                          const int32_t* row_token, const int32_t* row_slot, const float* row_w, int T, int D, int F,
                          int E, int k, float limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                          hipStream_t s) {
  const char* who = "grouped_experts_affine";
  if (bits == 2 && group == KC)
    return launch_grouped<KIND_Q2>(x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D, F, E, k,
                                   limit, y, workspace, workspace_bytes, s, who);
#define CACHALOT_GAFF(B, G)                                                                                      \
  if (bits == B && group == G)                                                                                   \
    return launch_grouped<aff_kind<B, G>>(x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D, F, \
                                          E, k, limit, y, workspace, workspace_bytes, s, who);
  CACHALOT_GAFF(2, 32) CACHALOT_GAFF(2, 64)
  CACHALOT_GAFF(3, 32) CACHALOT_GAFF(3, 64) CACHALOT_GAFF(3, 128)
  CACHALOT_GAFF(4, 32) CACHALOT_GAFF(4, 64) CACHALOT_GAFF(4, 128)
#undef CACHALOT_GAFF
  return fail(CACHALOT_EINVAL, "%s: %d-bit codes in groups of %d", who, bits, group);
}

}  // namespace cachalot

extern "C" int cachalot_permute(const int32_t* idx, const float* w, int T, int k, int E, int32_t* offsets,
                                int32_t* row_token, int32_t* row_slot, float* row_w, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(idx && w && offsets && row_token && row_slot && row_w, "permute: null pointer");
  CACHALOT_REQUIRE(T >= 1 && k >= 1 && (int64_t)T * k <= (1 << 30), "permute: T=%d k=%d", T, k);
  CACHALOT_REQUIRE(E >= 1 && E <= 1024, "permute: E=%d outside 1..1024", E);
  hipStream_t s = (hipStream_t)stream;
  if (T * k <= PERMUTE_THREADS) {
    hipLaunchKernelGGL(permute_small_kernel, dim3(1), dim3(PERMUTE_THREADS), 0, s, idx, w, T * k, k, E, offsets,
                       row_token, row_slot, row_w);
    return check_launch("permute_small_kernel");
  }
  hipLaunchKernelGGL(permute_scatter_kernel, dim3(E + 1), dim3(SCATTER_THREADS), 0, s, idx, w, T * k, k, E, offsets,
                     row_token, row_slot, row_w);
  return check_launch("permute_scatter_kernel");
}

extern "C" size_t cachalot_grouped_experts_workspace_bytes(int T, int k, int E, int D, int F) {
  (void)D;
  if (T <= 0 || k <= 0 || E <= 0 || F <= 0) return 0;
  return cachalot::grouped_ws(T, k, E, D, F).total;
}

// cachalot_permute followed by cachalot_grouped_experts_q2, with offsets / row_* as outputs;
// a batched decode of up to 1,024 routes permutes them inside its prep launch.
extern "C" int cachalot_grouped_experts_q2_routes(const uint16_t* x, const uint8_t* pool,
                                                  const cachalot_expert_layout* layout, const int32_t* slot_table,
                                                  const int32_t* idx, const float* w, int32_t* offsets,
                                                  int32_t* row_token, int32_t* row_slot, float* row_w, int T, int D,
                                                  int F, int E, int k, int group, float swiglu_limit, uint16_t* y,
                                                  void* workspace, size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(group == KC, "grouped_experts_q2: group_size %d (the bank format uses 128)", group);
  CACHALOT_REQUIRE(idx && w, "grouped_experts_q2: null routes");
  CACHALOT_REQUIRE((int64_t)T * k <= (1 << 30), "grouped_experts_q2: T=%d k=%d", T, k);
  return launch_grouped<KIND_Q2>(x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D, F, E, k,
                                 swiglu_limit, y, workspace, workspace_bytes, (hipStream_t)stream,
                                 "grouped_experts_q2", idx, w);
}

extern "C" int cachalot_grouped_experts_q2(const uint16_t* x, const uint8_t* pool,
                                           const cachalot_expert_layout* layout, const int32_t* slot_table,
                                           const int32_t* offsets, const int32_t* row_token, const int32_t* row_slot,
                                           const float* row_w, int T, int D, int F, int E, int k, int group,
                                           float swiglu_limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                                           cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(group == KC, "grouped_experts_q2: group_size %d (the bank format uses 128)", group);
  return launch_grouped<KIND_Q2>(x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D, F, E, k,
                                 swiglu_limit, y, workspace, workspace_bytes, (hipStream_t)stream,
                                 "grouped_experts_q2");
}

extern "C" int cachalot_grouped_experts_fp4(const uint16_t* x, const uint8_t* pool,
                                            const cachalot_expert_layout* layout, const int32_t* slot_table,
                                            const int32_t* offsets, const int32_t* row_token,
                                            const int32_t* row_slot, const float* row_w, int T, int D, int F, int E,
                                            int k, float swiglu_limit, uint16_t* y, void* workspace,
                                            size_t workspace_bytes, cachalot_stream_t stream) {
  using namespace cachalot;
  return launch_grouped<KIND_FP4>(x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D, F, E, k,
                                  swiglu_limit, y, workspace, workspace_bytes, (hipStream_t)stream,
                                  "grouped_experts_fp4");
}

extern "C" int cachalot_unpermute_combine(const uint16_t* y, const uint16_t* addend, int T, int k, int D,
                                          float* routed, uint16_t* out, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(y, "unpermute_combine: null pointer");
  CACHALOT_REQUIRE(routed || out, "unpermute_combine: no output requested");
  CACHALOT_REQUIRE(T >= 1 && k >= 1 && D >= 2 && D % 2 == 0, "unpermute_combine: T=%d k=%d D=%d", T, k, D);
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (D % 8 == 0 && k <= decode::KMAX && a16(y) && a16(addend) && a16(routed) && a16(out)) {
    const int64_t groups = (int64_t)T * D / 8;
    hipLaunchKernelGGL(combine8_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, (hipStream_t)stream, y,
                       addend, T, k, D, routed, out);
    return check_launch("combine8_kernel");
  }
  const int64_t pairs = (int64_t)T * D / 2;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, (hipStream_t)stream, y,
                     addend, T, k, D, routed, out);
  return check_launch("combine_kernel");
}
