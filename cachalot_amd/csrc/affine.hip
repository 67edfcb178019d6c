// Affine banks of any width the reference's bank tool writes: 2, 3 or 4 bits per
// code, groups of 32, 64 or 128 (benchmarks/build_affine_bank.py:266-267), bf16
// or fp16 scales and biases -- e.g. oMLX's oQ3e conversion, 3-bit codes in groups
// of 64 with fp16 scales (src/cachalot/model/expert_affine.py:1-10).  The 2-bit
// g128 bank keeps its matrix-core kernels (decode_q2_mx.hip, grouped.hip); every
// other width runs here.
//
// Layout (MLX's, benchmarks/quant_affine.py:69-105): a row's codes are one
// little-endian bit stream, code i at bits [i b, (i + 1) b), words filled from
// the least significant bit, nothing padded; a group of G codes spans G b / 32
// whole words, so groups start on word boundaries.  K is padded to whole groups
// with zero codes.  Value = s q + b per group (fp32 from the stored scale type).
//
// Arithmetic: the reference's group formula s * sum(x q) + b * sum(x)
// (minimax/codes_qmv.py:86-100) with fp32 sums; the SwiGLU expert's rounding
// points are those of the 2-bit path: g = bf16(x W1), u = bf16(x W3), clamp,
// h = bf16(silu(g) u w), y_e = bf16(h W2), routed = 0 + y_0 + .. + y_{k-1} in
// route order (expert_affine.py:65-81,117-152), out = bf16(routed + addend).
//
// Kernels (VALU GEMV; one lane per group of a weight row, the wave's lanes over
// the row's groups, then a butterfly):
//   aff_gate_up_kernel  one workgroup = 16 rows of W1 and of W3 for one expert
//     and up to TB token rows (decode: the routed expert's one token, selected on
//     the device when the router's scores are given); writes h rows (bf16, padded
//     to whole groups with zeros).
//   aff_down_kernel     one workgroup = 16 rows of W2: decode, all k experts in
//     route order summed into routed / out; grouped, one expert's TB rows into
//     y[token, slot, :].
//   aff_dequant_kernel  dense fp32 weights (bit-exact checks).
#include <algorithm>

#include "decode_common.h"
#include "router_launch.h"
#include "mx_tile.h"

namespace cachalot {

// decode_affine_mx.hip
bool affine_mx_supported(int bits, int group, int D, int F, int k);
size_t affine_mx_hidden_bytes(int k, int D, int F);
int launch_affine_mx(const uint16_t* x, bool planes_ready, uint8_t* hid, uint8_t* xplanes, const uint8_t* pool,
                     const decode::Layout& L, const decode::ExpertSource& src, int32_t* ws_slots, float* ws_w, int D,
                     int F, int k, int bits, int group, float limit, const uint16_t* addend, float* routed,
                     uint16_t* out, hipStream_t s);

// grouped.hip: the other widths on the bf16-MFMA grouped kernels
size_t grouped_affine_ws_bytes(int T, int k, int E, int D, int F);
int launch_grouped_affine(int bits, int group, const uint16_t* x, const uint8_t* pool,
                          const cachalot_expert_layout* layout, const int32_t* slot_table, const int32_t* offsets,
                          const int32_t* row_token, const int32_t* row_slot, const float* row_w, int T, int D, int F,
                          int E, int k, float limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                          hipStream_t s);

namespace aff {

using namespace decode;

constexpr int THREADS = 256;
constexpr int TB = 4;            // token rows per grouped tile
constexpr int MAX_K = 8192;      // D, F (padded) <= MAX_K

// Code i (0 <= i < G) of a group whose WORDS = G * BITS / 32 words are w.
template <int BITS>
__device__ __forceinline__ uint32_t code_of(const uint32_t* w, int i) {
  const int bit = i * BITS, wi = bit >> 5, sh = bit & 31;
  uint32_t v = w[wi] >> sh;
  if (sh + BITS > 32) v |= w[wi + 1] << (32 - sh);
  return v & ((1u << BITS) - 1u);
}

// Rows are read in units of 32 codes -- BITS whole words -- dealt to the lanes
// (unit u to lane u % 64); unit u lies in group 32 u / G.  A lane's value for a
// row is the sum over its units of s * sum(x q), plus b * sum(x) for each group
// whose first unit it holds (sum(x) per group precomputed once per activation
// row); the wave butterfly then adds the lanes.  All of a wave's rows are loaded
// before any is used, so their loads are in flight together.
constexpr int UNIT = 32;

template <int BITS>
struct Unit {
  uint32_t w[BITS];
};

template <int BITS>
__device__ __forceinline__ Unit<BITS> load_unit(const uint8_t* row, int u) {
  Unit<BITS> r;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(row) + (size_t)u * BITS;
  if constexpr (BITS == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else if constexpr (BITS == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    r.w[0] = v.x;
    r.w[1] = v.y;
    r.w[2] = v.z;
    r.w[3] = v.w;
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) r.w[i] = p[i];
  }
  return r;
}

// R rows' units (UPL per lane), scales and group biases, loaded together.
template <int BITS, int G, int R, int UPL>
struct Rows {
  Unit<BITS> w[R][UPL];
  float s[R][UPL], b[R][UPL];
};

template <int BITS, int G, int R, int UPL>
__device__ __forceinline__ void load_rows(const uint8_t* const (&wrow)[R], const uint16_t* const (&srow)[R],
                                          const uint16_t* const (&brow)[R], bool f16, int nunits,
                                          Rows<BITS, G, R, UPL>& o) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = min(lane + 64 * j, nunits - 1);
      o.w[r][j] = load_unit<BITS>(wrow[r], u);
      const int g = u * UNIT / G;
      o.s[r][j] = scale_bits_to_f32(srow[r][g], f16);
      o.b[r][j] = scale_bits_to_f32(brow[r][g], f16);
    }
}

// out[r] = the rows' dot products with one activation row x (fp32, LDS), xsum its
// per-group sums; returned to every lane.
template <int BITS, int G, int R, int UPL>
__device__ __forceinline__ void dot_rows(const Rows<BITS, G, R, UPL>& o, int nunits, const float* x,
                                         const float* xsum, float (&out)[R]) {
  const int lane = threadIdx.x & 63;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (u >= nunits) break;
    const float4* xv = reinterpret_cast<const float4*>(x + u * UNIT);
    const bool first = (u * UNIT) % G == 0;
    const float gs = first ? xsum[u * UNIT / G] : 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float d = 0.0f;
#pragma unroll
      for (int i4 = 0; i4 < UNIT / 4; ++i4) {
        const float4 xx = xv[i4];
        d = __builtin_fmaf(xx.x, (float)code_of<BITS>(o.w[r][j].w, 4 * i4), d);
        d = __builtin_fmaf(xx.y, (float)code_of<BITS>(o.w[r][j].w, 4 * i4 + 1), d);
        d = __builtin_fmaf(xx.z, (float)code_of<BITS>(o.w[r][j].w, 4 * i4 + 2), d);
        d = __builtin_fmaf(xx.w, (float)code_of<BITS>(o.w[r][j].w, 4 * i4 + 3), d);
      }
      acc[r] = acc[r] + (o.s[r][j] * d + o.b[r][j] * gs);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = wave_sum(acc[r]);
}

// Per-group sums of NT activation rows (x [t][ld], padding zero) into xsum [t][ld / G]:
// G / 16 consecutive threads per group, 16 values each, then a butterfly inside the
// thread group (every thread of the workgroup takes part in every pass).
template <int G>
__device__ __forceinline__ void group_sums(const float* x, int ld, int nt, float* xsum) {
  constexpr int P = G / 16;   // threads per group (2, 4 or 8: aligned inside a quad pair)
  const int ng = ld / G, total = nt * ng * P;
  for (int i0 = 0; i0 < total; i0 += blockDim.x) {
    const int i = i0 + threadIdx.x;
    const int q = min(i, total - 1), grp = q / P, part = q - grp * P;
    const int t = grp / ng, g = grp - t * ng;
    const float4* p = reinterpret_cast<const float4*>(x + t * ld + g * G + 16 * part);
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 f = p[v];
      sum = sum + f.x + f.y + f.z + f.w;
    }
    sum = sum + __uint_as_float(xor1_u32(__float_as_uint(sum)));
    if constexpr (P >= 4) sum = sum + __uint_as_float(xor2_u32(__float_as_uint(sum)));
    if constexpr (P >= 8) sum = sum + __uint_as_float(mirror8_u32(__float_as_uint(sum)));
    if (i < total && part == 0) xsum[grp] = sum;
  }
}

// Where a gate/up or down workgroup finds its rows.  Decode: route e of one
// token (idx / w given, or selected from the scores).  Grouped: a tile of up to TB
// expert-major rows (offsets, row_token, row_w of cachalot_permute).
struct Args {
  const uint16_t* x;        // [T, D] bf16
  const uint8_t* pool;
  Layout L;
  ExpertSource src;         // decode
  int D, F, k;
  float limit;
  uint16_t* h;              // [rows][Fp] bf16 (decode: rows = k)
  int32_t* ws_slots;
  float* ws_w;
  // grouped
  const int32_t* slot_table;
  const int32_t* offsets;
  const int32_t* row_token;
  const int32_t* row_slot;
  const float* row_w;
  const int32_t* tile_prefix;   // [E + 1] tiles before expert e
  int E, max_tiles;
  // outputs
  const uint16_t* addend;
  float* routed;
  uint16_t* out;
  uint16_t* y;              // grouped: [T, k, D]
};

// Tile t of the grouped tile list: its expert (binary search of tile_prefix) and first row.
__device__ __forceinline__ bool tile_of(const Args& a, int t, int& e, int& r0, int& nr) {
  if (t >= a.tile_prefix[a.E]) return false;
  int lo = 0, hi = a.E;   // tile_prefix[lo] <= t < tile_prefix[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.tile_prefix[mid] <= t) lo = mid;
    else hi = mid;
  }
  e = lo;
  r0 = a.offsets[e] + (t - a.tile_prefix[e]) * TB;
  nr = min(TB, a.offsets[e + 1] - r0);
  return true;
}

// tile_prefix[e] = sum over e' < e of ceil(rows_e' / TB); one workgroup of 1024 threads.
__global__ void __launch_bounds__(1024) aff_tiles_kernel(const int32_t* __restrict__ offsets, int E,
                                                         int32_t* __restrict__ tile_prefix) {
  __shared__ int part[1024];
  const int t = threadIdx.x;
  part[t] = t < E ? (offsets[t + 1] - offsets[t] + TB - 1) / TB : 0;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {   // inclusive scan
    const int v = t >= d ? part[t - d] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  if (t < E) tile_prefix[t + 1] = part[t];
  if (t == 0) tile_prefix[0] = 0;
}

// Zero y rows of the dropped routes (rows offsets[E] .. n - 1): one workgroup per row.
__global__ void __launch_bounds__(256) aff_drop_kernel(const int32_t* __restrict__ offsets, int E, int n,
                                                       const int32_t* __restrict__ row_token,
                                                       const int32_t* __restrict__ row_slot, int k, int D,
                                                       uint16_t* __restrict__ y) {
  const int r = blockIdx.x;
  if (r < offsets[E] || r >= n) return;
  uint16_t* dst = y + ((size_t)row_token[r] * k + row_slot[r]) * D;
  for (int i = threadIdx.x; i < D; i += 256) dst[i] = 0;
}

// grid.x = k * F / 16 (decode) or max_tiles * F / 16 (grouped).
template <int BITS, int G, int UPL, bool GROUPED>
__global__ void __launch_bounds__(THREADS) aff_gate_up_kernel(Args a) {
  extern __shared__ float xs[];   // [TB or 1][Dp] fp32
  __shared__ float xsum[TB * MAX_K / UNIT];
  __shared__ int top_i[KMAX], top_s[KMAX];
  __shared__ float top_v[KMAX], top_w[KMAX];
  __shared__ float red[2][16][TB];
  __shared__ int s_slot;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int FT = a.F / 16, Dp = (a.D + G - 1) / G * G, Fp = (a.F + G - 1) / G * G;
  const int unit = blockIdx.x / FT, tile = blockIdx.x - unit * FT, row0 = tile * 16;
  int e, r0 = 0, nr = 1, slot;
  if constexpr (GROUPED) {
    if (!tile_of(a, unit, e, r0, nr)) return;
    slot = a.slot_table[e];
  } else {
    e = unit;
    if (wave == 0) {   // the expert's slot (the top-k itself, given scores) while the x rows are staged
      const int sl = route_slot(a.src, a.ws_slots, e, top_i, top_v, top_s);
      if (lane == 0) s_slot = sl;
    }
  }
  const int NT = GROUPED ? nr : 1;
  // activation rows into LDS (fp32; the padding past D is zero), 8 values per thread and step
  for (int t = 0; t < NT; ++t) {
    const int tok = GROUPED ? a.row_token[r0 + t] : 0;
    const uint16_t* xr = a.x + (size_t)tok * a.D;
    for (int i = 8 * tid; i < Dp; i += 8 * THREADS) {
      float v[8];
      if (i + 8 <= a.D) {
        const uint4 raw = *reinterpret_cast<const uint4*>(xr + i);
        const uint32_t ww[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[2 * q] = __uint_as_float(ww[q] << 16);
          v[2 * q + 1] = __uint_as_float(ww[q] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = i + q < a.D ? bf16_to_f32(xr[i + q]) : 0.0f;
      }
      float4* d = reinterpret_cast<float4*>(xs + t * Dp + i);
      d[0] = make_float4(v[0], v[1], v[2], v[3]);
      d[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  __syncthreads();
  if constexpr (!GROUPED) slot = s_slot;
  const int Gn = Dp / G;
  if (slot >= 0) {
    const uint8_t* base = a.pool + (int64_t)slot * a.L.record_bytes;
    const int wb = Dp * BITS / 8;   // bytes per weight row
    // wave w: rows 4w .. 4w + 3 of W1 (r < 4) and of W3 (r >= 4); grouped tiles (several
    // activation rows) take the two matrices in turn, so fewer rows stay live
    constexpr int R = GROUPED ? 4 : 8;
#pragma unroll
    for (int pass = 0; pass < 8 / R; ++pass) {
      const uint8_t* wrow[R];
      const uint16_t* srow[R];
      const uint16_t* brow[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int rr = pass * R + r;
        const int n = row0 + 4 * wave + (rr & 3), tq = rr < 4 ? 0 : 6;
        wrow[r] = base + a.L.off[tq] + (int64_t)n * wb;
        srow[r] = reinterpret_cast<const uint16_t*>(base + a.L.off[tq + 1]) + (int64_t)n * Gn;
        brow[r] = reinterpret_cast<const uint16_t*>(base + a.L.off[tq + 2]) + (int64_t)n * Gn;
      }
      Rows<BITS, G, R, UPL> rw;
      load_rows<BITS, G, R, UPL>(wrow, srow, brow, a.L.f16, Dp / UNIT, rw);
      if (pass == 0) {   // the group sums while the first rows' loads are in flight
        group_sums<G>(xs, Dp, NT, xsum);
        __syncthreads();
      }
      for (int t = 0; t < NT; ++t) {
        float v[R];
        dot_rows<BITS, G, R, UPL>(rw, Dp / UNIT, xs + t * Dp, xsum + t * Gn, v);
        if (lane == 0)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int rr = pass * R + r;
            red[rr >> 2][4 * wave + (rr & 3)][t] = v[r];
          }
      }
    }
  }
  __syncthreads();
  // epilogue: thread (t, j) -> token row t, weight row row0 + j
  if (tid < 16 * TB) {
    const int j = tid & 15, t = tid >> 4;
    float wexp = 0.0f;
    if constexpr (!GROUPED) {
      if (t == 0) wexp = route_finish(a.src, a.ws_w, e, tile, top_v, top_w, top_i, blockIdx.x == 0);
      if (tid == 0 && (a.src.idx || a.src.scores) && tile == 0) a.ws_slots[e] = slot;
    }
    if (t < NT) {
      const int hr = GROUPED ? r0 + t : e;
      if constexpr (GROUPED) wexp = a.row_w[hr];
      float hv = 0.0f;
      if (slot >= 0) {
        float g = round_bf16(red[0][j][t]), u = round_bf16(red[1][j][t]);
        if (a.limit > 0.0f) {
          u = fminf(fmaxf(u, -a.limit), a.limit);
          g = fminf(g, a.limit);
        }
        hv = (silu_f32(g) * u) * wexp;
      }
      uint16_t* hrow = a.h + (size_t)hr * Fp;
      hrow[row0 + j] = f32_to_bf16(hv);
      if (tile == FT - 1)   // the padding past F: zeros
        for (int i = a.F + j; i < Fp; i += 16) hrow[i] = 0;
    }
  }
}

// grid.x = D / 16 (decode) or (D / 16) x max_tiles (grouped: blockIdx.y = tile).
template <int BITS, int G, int UPL, bool GROUPED>
__global__ void __launch_bounds__(THREADS) aff_down_kernel(Args a) {
  extern __shared__ float hs[];   // [TB][Fp] fp32
  __shared__ float hsum[TB * MAX_K / UNIT];
  __shared__ float yv[KMAX][16][TB];
  __shared__ int slots[KMAX];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int Fp = (a.F + G - 1) / G * G, Gn = Fp / G;
  const int row0 = blockIdx.x * 16;
  int e0 = 0, r0 = 0, nr = 1, ne = a.k;
  if constexpr (GROUPED) {
    if (!tile_of(a, blockIdx.y, e0, r0, nr)) return;
    ne = 1;
  }
  if (tid < ne) slots[tid] = GROUPED ? a.slot_table[e0] : expert_slot(a.src, a.ws_slots, tid);
  for (int x = 0; x < ne; ++x) {
    const int NT = GROUPED ? nr : 1;
    __syncthreads();   // slots written; the previous expert's h no longer read
    const int slot = slots[x];
    // this expert's rows first, so their loads fly while h is staged and summed
    Rows<BITS, G, 4, UPL> rw;
    if (slot >= 0) {
      const uint8_t* base = a.pool + (int64_t)slot * a.L.record_bytes;
      const int wb = Fp * BITS / 8;
      const uint8_t* wrow[4];
      const uint16_t* srow[4];
      const uint16_t* brow[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = row0 + 4 * wave + r;
        wrow[r] = base + a.L.off[3] + (int64_t)n * wb;
        srow[r] = reinterpret_cast<const uint16_t*>(base + a.L.off[4]) + (int64_t)n * Gn;
        brow[r] = reinterpret_cast<const uint16_t*>(base + a.L.off[5]) + (int64_t)n * Gn;
      }
      load_rows<BITS, G, 4, UPL>(wrow, srow, brow, a.L.f16, Fp / UNIT, rw);
    }
    for (int t = 0; t < NT; ++t) {
      const uint16_t* hrow = a.h + (size_t)(GROUPED ? r0 + t : x) * Fp;
      for (int i = 8 * tid; i < Fp; i += 8 * THREADS) {   // padded with zeros by the gate/up kernel
        const uint4 raw = *reinterpret_cast<const uint4*>(hrow + i);
        const uint32_t ww[4] = {raw.x, raw.y, raw.z, raw.w};
        float4* d = reinterpret_cast<float4*>(hs + t * Fp + i);
        d[0] = make_float4(__uint_as_float(ww[0] << 16), __uint_as_float(ww[0] & 0xffff0000u),
                           __uint_as_float(ww[1] << 16), __uint_as_float(ww[1] & 0xffff0000u));
        d[1] = make_float4(__uint_as_float(ww[2] << 16), __uint_as_float(ww[2] & 0xffff0000u),
                           __uint_as_float(ww[3] << 16), __uint_as_float(ww[3] & 0xffff0000u));
      }
    }
    __syncthreads();
    group_sums<G>(hs, Fp, NT, hsum);
    __syncthreads();
    if (slot >= 0) {
      for (int t = 0; t < NT; ++t) {
        float v[4];
        dot_rows<BITS, G, 4, UPL>(rw, Fp / UNIT, hs + t * Fp, hsum + t * Gn, v);
        if (lane == 0)
#pragma unroll
          for (int r = 0; r < 4; ++r) yv[x][4 * wave + r][t] = v[r];
      }
    } else if (lane == 0) {
      for (int r = 0; r < 4; ++r)
        for (int t = 0; t < TB; ++t) yv[x][4 * wave + r][t] = 0.0f;
    }
  }
  __syncthreads();
  if constexpr (GROUPED) {
    if (tid < 16 * TB) {
      const int j = tid & 15, t = tid >> 4;
      if (t < nr) {
        const int rr = r0 + t;
        a.y[((size_t)a.row_token[rr] * a.k + a.row_slot[rr]) * a.D + row0 + j] = f32_to_bf16(yv[0][j][t]);
      }
    }
  } else if (tid < 16) {
    const int n = row0 + tid;
    float total = 0.0f;
    for (int x = 0; x < a.k; ++x) total = total + round_bf16(yv[x][tid][0]);
    if (a.routed) a.routed[n] = total;
    if (a.out) a.out[n] = f32_to_bf16(a.addend ? total + bf16_to_f32(a.addend[n]) : total);
  }
}

// One thread per 32-code unit of a row: w [N, row_words], scales / biases [N, groups].
template <int BITS, int G>
__global__ void __launch_bounds__(256) aff_dequant_kernel(const uint32_t* __restrict__ w,
                                                          const uint16_t* __restrict__ scales,
                                                          const uint16_t* __restrict__ biases, int N, int K,
                                                          int row_words, int groups, bool f16,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nu = (K + UNIT - 1) / UNIT;
  if (i >= (int64_t)N * nu) return;
  const int64_t n = i / nu;
  const int u = (int)(i - n * nu), g = u * UNIT / G;
  const Unit<BITS> c = load_unit<BITS>(reinterpret_cast<const uint8_t*>(w + n * row_words), u);
  const float s = scale_bits_to_f32(scales[n * groups + g], f16), b = scale_bits_to_f32(biases[n * groups + g], f16);
#pragma unroll
  for (int t = 0; t < UNIT; ++t) {
    const int k = u * UNIT + t;
    if (k < K) out[n * K + k] = s * (float)code_of<BITS>(c.w, t) + b;
  }
}

// ------------------------------------------------------------------ host ---
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

bool supported(int bits, int group) {
  return (bits == 2 || bits == 3 || bits == 4) && (group == 32 || group == 64 || group == 128);
}

template <template <int, int> class Fn, typename... A>
int dispatch(int bits, int group, A... args) {
#define CACHALOT_AFF(B, G) \
  if (bits == B && group == G) return Fn<B, G>::run(args...);
  CACHALOT_AFF(2, 32) CACHALOT_AFF(2, 64) CACHALOT_AFF(2, 128)
  CACHALOT_AFF(3, 32) CACHALOT_AFF(3, 64) CACHALOT_AFF(3, 128)
  CACHALOT_AFF(4, 32) CACHALOT_AFF(4, 64) CACHALOT_AFF(4, 128)
#undef CACHALOT_AFF
  return fail(CACHALOT_EINVAL, "affine: %d-bit codes in groups of %d are not a bank format (bits 2/3/4, group "
              "32/64/128)", bits, group);
}

template <int BITS, int G, int UPL>
int run_decode(const Args& a, bool grouped, hipStream_t s) {
  const int Dp = (a.D + G - 1) / G * G, Fp = (a.F + G - 1) / G * G;
  const int nt = grouped ? TB : 1;
  const size_t lds_gu = (size_t)nt * Dp * 4, lds_dn = (size_t)nt * Fp * 4;
  const void* kgu = grouped ? reinterpret_cast<const void*>(aff_gate_up_kernel<BITS, G, UPL, true>)
                            : reinterpret_cast<const void*>(aff_gate_up_kernel<BITS, G, UPL, false>);
  const void* kdn = grouped ? reinterpret_cast<const void*>(aff_down_kernel<BITS, G, UPL, true>)
                            : reinterpret_cast<const void*>(aff_down_kernel<BITS, G, UPL, false>);
  if (hipFuncSetAttribute(kgu, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_gu) != hipSuccess ||
      hipFuncSetAttribute(kdn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_dn) != hipSuccess)
    return fail(CACHALOT_EHIP, "affine: cannot grant %zu / %zu bytes of LDS", lds_gu, lds_dn);
  if (grouped) {
    hipLaunchKernelGGL((aff_gate_up_kernel<BITS, G, UPL, true>), dim3((unsigned)(a.max_tiles * (a.F / 16))),
                       dim3(THREADS), lds_gu, s, a);
    if (int rc = check_launch("aff_gate_up_kernel")) return rc;
    hipLaunchKernelGGL((aff_down_kernel<BITS, G, UPL, true>), dim3((unsigned)(a.D / 16), (unsigned)a.max_tiles),
                       dim3(THREADS), lds_dn, s, a);
    return check_launch("aff_down_kernel");
  }
  hipLaunchKernelGGL((aff_gate_up_kernel<BITS, G, UPL, false>), dim3((unsigned)(a.k * (a.F / 16))), dim3(THREADS),
                     lds_gu, s, a);
  if (int rc = check_launch("aff_gate_up_kernel")) return rc;
  hipLaunchKernelGGL((aff_down_kernel<BITS, G, UPL, false>), dim3((unsigned)(a.D / 16)), dim3(THREADS), lds_dn, s,
                     a);
  return check_launch("aff_down_kernel");
}

// UPL = units per lane for the longer K: 2 up to 4096, 4 up to MAX_K.
template <int BITS, int G>
struct Decode {
  static int run(const Args& a, bool grouped, hipStream_t s) {
    const int kmax = std::max((a.D + G - 1) / G * G, (a.F + G - 1) / G * G);
    return kmax <= 64 * 2 * UNIT ? run_decode<BITS, G, 2>(a, grouped, s) : run_decode<BITS, G, 4>(a, grouped, s);
  }
};

template <int BITS, int G>
struct Dequant {
  static int run(const uint32_t* w, const uint16_t* sc, const uint16_t* bi, int N, int K, int row_words, int groups,
                 bool f16, float* out, hipStream_t s) {
    const int64_t total = (int64_t)N * ((K + UNIT - 1) / UNIT);
    hipLaunchKernelGGL((aff_dequant_kernel<BITS, G>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, w, sc,
                       bi, N, K, row_words, groups, f16, out);
    return check_launch("aff_dequant_kernel");
  }
};

int check_shape(const char* who, int D, int F, int bits, int group) {
  if (!supported(bits, group))
    return fail(CACHALOT_EINVAL, "%s: %d-bit codes in groups of %d are not a bank format (bits 2/3/4, group "
                "32/64/128)", who, bits, group);
  CACHALOT_REQUIRE(D % 16 == 0 && D >= 16 && (D + group - 1) / group * group <= MAX_K,
                   "%s: D=%d must be a multiple of 16 up to %d", who, D, MAX_K);
  CACHALOT_REQUIRE(F % 16 == 0 && F >= 16 && (F + group - 1) / group * group <= MAX_K,
                   "%s: F=%d must be a multiple of 16 up to %d", who, F, MAX_K);
  return CACHALOT_OK;
}

size_t hidden_bytes(int rows, int F) { return align256((size_t)rows * ((F + 127) / 128 * 128) * 2); }

// The decode workspace's hidden region: the VALU kernels' bf16 h rows or the
// matrix-core kernels' plane blocks (h, then x), whichever is larger.
size_t decode_hidden_bytes(int k, int D, int F) {
  return std::max(hidden_bytes(k, F), affine_mx_hidden_bytes(k, D, F));
}

// The VALU kernels stay selectable for the widths the matrix-core kernels take
// (CACHALOT_AFFINE_VALU=1), so that the tests hold both to the oracle.
bool valu_requested() {
  const char* env = getenv("CACHALOT_AFFINE_VALU");
  return env && env[0] == '1';
}

int decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout, ExpertSource src,
           const RouterCall* router, int D, int F, int k, int bits, int group, float limit, const uint16_t* addend,
           float* routed, uint16_t* out, void* workspace, size_t workspace_bytes, hipStream_t s) {
  CACHALOT_REQUIRE(pool && layout && src.slot_table && x, "moe_decode_affine: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_affine: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_affine: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(src.E >= 1 && src.E <= 1024, "moe_decode_affine: E=%d outside 1..1024", src.E);
  if (int rc = check_shape("moe_decode_affine", D, F, bits, group)) return rc;
  const WsOffsets wo = ws_offsets(decode_hidden_bytes(k, D, F));
  if (workspace == nullptr || workspace_bytes < wo.total)
    return fail(CACHALOT_ESPACE, "moe_decode_affine: workspace %zu < %zu bytes", workspace_bytes, wo.total);
  Args a{};
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  if (int rc = make_layout(layout, 9, used, a.L, "moe_decode_affine")) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  if (affine_mx_supported(bits, group, D, F, k) && !valu_requested()) {
    // the block-scaled matrix-core kernels (decode_affine_mx.hip): h planes, then x planes,
    // which the router launch writes when there is one
    uint8_t* hid = ws + wo.hidden;
    uint8_t* xplanes = hid + align256((size_t)k * ((F + 127) / 128) * mx::PB_BYTES);
    if (router) {
      if (int rc = launch_router_scores(x, router->gate_weight, 1, D, src.E, router->gate_temp, router->score_fn,
                                        router->scores, s, nullptr, xplanes))
        return rc;
      src = route_source(src, *router);
    }
    return launch_affine_mx(x, router != nullptr, hid, xplanes, pool, a.L, src,
                            reinterpret_cast<int32_t*>(ws + wo.slots), reinterpret_cast<float*>(ws + wo.weights), D,
                            F, k, bits, group, limit, addend, routed, out, s);
  }
  if (router) {
    if (int rc = launch_router_scores(x, router->gate_weight, 1, D, src.E, router->gate_temp, router->score_fn,
                                      router->scores, s))
      return rc;
    src = route_source(src, *router);
  }
  a.x = x;
  a.pool = pool;
  a.src = src;
  a.D = D;
  a.F = F;
  a.k = k;
  a.limit = limit;
  a.h = reinterpret_cast<uint16_t*>(ws + wo.hidden);
  a.ws_slots = reinterpret_cast<int32_t*>(ws + wo.slots);
  a.ws_w = reinterpret_cast<float*>(ws + wo.weights);
  a.addend = addend;
  a.routed = routed;
  a.out = out;
  return dispatch<Decode>(bits, group, a, false, s);
}

}  // namespace aff
}  // namespace cachalot

using namespace cachalot;

extern "C" size_t cachalot_moe_decode_affine_workspace_bytes(int D, int F, int k) {
  if (D <= 0 || F <= 0 || k <= 0 || k > decode::KMAX) return 0;
  return decode::ws_offsets(aff::decode_hidden_bytes(k, D, F)).total;
}

extern "C" int cachalot_moe_decode_affine(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout,
                                          const int32_t* slot_table, const int32_t* idx, const float* w, int D, int F,
                                          int E, int k, int bits, int group, float swiglu_limit,
                                          const uint16_t* addend, float* routed, uint16_t* out, void* workspace,
                                          size_t workspace_bytes, cachalot_stream_t stream) {
  CACHALOT_REQUIRE(idx && w, "moe_decode_affine: null routes");
  decode::ExpertSource src{slot_table, idx, w, E};
  return aff::decode(x, pool, layout, src, nullptr, D, F, k, bits, group, swiglu_limit, addend, routed, out,
                     workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cachalot_moe_layer_decode_affine(const uint16_t* x, const uint16_t* gate_weight,
                                                const float* gate_bias, int E, int k, int score_fn, float gate_temp,
                                                float route_scale, int norm, int order, const uint8_t* pool,
                                                const cachalot_expert_layout* layout, const int32_t* slot_table, int D,
                                                int F, int bits, int group, float swiglu_limit,
                                                const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                                float* routed, uint16_t* out, void* workspace,
                                                size_t workspace_bytes, cachalot_stream_t stream) {
  CACHALOT_REQUIRE(gate_weight && gate_bias && scores, "moe_layer_decode_affine: null router pointer");
  CACHALOT_REQUIRE(D % 128 == 0, "moe_layer_decode_affine: D=%d must be a multiple of 128", D);
  CACHALOT_REQUIRE(score_fn == CACHALOT_SCORE_SQRT_SOFTPLUS || score_fn == CACHALOT_SCORE_SIGMOID,
                   "moe_layer_decode_affine: unknown score function %d", score_fn);
  CACHALOT_REQUIRE(order == CACHALOT_ORDER_ASCENDING || order == CACHALOT_ORDER_RANK,
                   "moe_layer_decode_affine: unknown order %d", order);
  CACHALOT_REQUIRE(gate_temp != 0.0f, "moe_layer_decode_affine: gate_temp must be non-zero");
  CACHALOT_REQUIRE(k >= 1 && k <= E && E <= 1024, "moe_layer_decode_affine: invalid topk=%d for %d experts", k, E);
  decode::ExpertSource src{slot_table, nullptr, nullptr, E};
  RouterCall rt{gate_weight, score_fn, gate_temp, scores, {}};
  rt.tail = decode::RouteTail{gate_bias, slot_table, idx_out, w_out, nullptr, nullptr, nullptr, E, k, order, norm,
                              route_scale};
  return aff::decode(x, pool, layout, src, &rt, D, F, k, bits, group, swiglu_limit, addend, routed, out, workspace,
                     workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t cachalot_grouped_experts_affine_workspace_bytes(int T, int k, int E, int D, int F) {
  if (T <= 0 || k <= 0 || E <= 0 || D <= 0 || F <= 0) return 0;
  return std::max(aff::align256((size_t)(E + 1) * 4) + aff::hidden_bytes(T * k, F),
                  grouped_affine_ws_bytes(T, k, E, D, F));
}

extern "C" int cachalot_grouped_experts_affine(const uint16_t* x, const uint8_t* pool,
                                               const cachalot_expert_layout* layout, const int32_t* slot_table,
                                               const int32_t* offsets, const int32_t* row_token,
                                               const int32_t* row_slot, const float* row_w, int T, int D, int F,
                                               int E, int k, int bits, int group, float swiglu_limit, uint16_t* y,
                                               void* workspace, size_t workspace_bytes, cachalot_stream_t stream) {
  CACHALOT_REQUIRE(x && pool && layout && slot_table && offsets && row_token && row_slot && row_w && y,
                   "grouped_experts_affine: null pointer");
  CACHALOT_REQUIRE(T >= 1 && k >= 1 && E >= 1 && E <= 1024, "grouped_experts_affine: T=%d k=%d E=%d", T, k, E);
  if (int rc = aff::check_shape("grouped_experts_affine", D, F, bits, group)) return rc;
  const size_t need = cachalot_grouped_experts_affine_workspace_bytes(T, k, E, D, F);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CACHALOT_ESPACE, "grouped_experts_affine: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  // the bf16 matrix cores (grouped.hip) where their tiling fits; the VALU kernels otherwise
  // and with CACHALOT_AFFINE_VALU=1
  if (D % 128 == 0 && F % 64 == 0 && D <= 8192 && F <= 8192 && k <= decode::KMAX && !aff::valu_requested())
    return launch_grouped_affine(bits, group, x, pool, layout, slot_table, offsets, row_token, row_slot, row_w, T, D,
                                 F, E, k, swiglu_limit, y, workspace, workspace_bytes, s);
  aff::Args a{};
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  if (int rc = decode::make_layout(layout, 9, used, a.L, "grouped_experts_affine")) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* tp = reinterpret_cast<int32_t*>(ws);
  // rows of dropped routes (offsets[E] ..) get zero y rows, by a kernel (no memset
  // node, so the call can be captured in a graph)
  hipLaunchKernelGGL(aff::aff_drop_kernel, dim3((unsigned)(T * k)), dim3(256), 0, s, offsets, E, T * k, row_token,
                     row_slot, k, D, y);
  if (int rc = check_launch("aff_drop_kernel")) return rc;
  hipLaunchKernelGGL(aff::aff_tiles_kernel, dim3(1), dim3(1024), 0, s, offsets, E, tp);
  if (int rc = check_launch("aff_tiles_kernel")) return rc;
  a.x = x;
  a.pool = pool;
  a.D = D;
  a.F = F;
  a.k = k;
  a.limit = swiglu_limit;
  a.h = reinterpret_cast<uint16_t*>(ws + aff::align256((size_t)(E + 1) * 4));
  a.slot_table = slot_table;
  a.offsets = offsets;
  a.row_token = row_token;
  a.row_slot = row_slot;
  a.row_w = row_w;
  a.tile_prefix = tp;
  a.E = E;
  a.max_tiles = (T * k + aff::TB - 1) / aff::TB + E;
  a.y = y;
  return aff::dispatch<aff::Decode>(bits, group, a, true, s);
}

extern "C" int cachalot_dequant_affine(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                                       int row_words, int groups, int group, int bits, int scale_dtype, float* out,
                                       cachalot_stream_t stream) {
  CACHALOT_REQUIRE(w && scales && biases && out, "dequant_affine: null pointer");
  CACHALOT_REQUIRE(aff::supported(bits, group), "dequant_affine: %d-bit codes in groups of %d", bits, group);
  CACHALOT_REQUIRE(N >= 1 && K >= 1, "dequant_affine: N=%d K=%d", N, K);
  CACHALOT_REQUIRE(scale_dtype == CACHALOT_SCALE_BF16 || scale_dtype == CACHALOT_SCALE_F16,
                   "dequant_affine: scale_dtype %d (0 = bf16, 1 = fp16)", scale_dtype);
  const int gk = (K + group - 1) / group;
  CACHALOT_REQUIRE(groups >= gk && row_words >= gk * group * bits / 32,
                   "dequant_affine: row_words %d / groups %d too small for K=%d", row_words, groups, K);
  return aff::dispatch<aff::Dequant>(bits, group, w, scales, biases, N, K, row_words, groups,
                                     scale_dtype == CACHALOT_SCALE_F16, out, (hipStream_t)stream);
}
