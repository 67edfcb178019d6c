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
#include "decode_common.h"
#include "router_launch.h"

namespace cachalot {
namespace aff {

using namespace decode;

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
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

// s * sum(x q) + b * sum(x) over one group; x: the group's G values (fp32, LDS).
template <int BITS, int G>
__device__ __forceinline__ float group_value(const uint32_t (&w)[G * BITS / 32], const float* x, float s, float b) {
  float sxq = 0.0f, sx = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float xi = x[i];
    sxq = sxq + xi * (float)code_of<BITS>(w, i);
    sx = sx + xi;
  }
  return s * sxq + b * sx;
}

template <int BITS, int G>
__device__ __forceinline__ void load_group(const uint8_t* row, int g, uint32_t (&w)[G * BITS / 32]) {
  constexpr int WORDS = G * BITS / 32;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(row) + (size_t)g * WORDS;
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int q = 0; q < WORDS / 4; ++q) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[q];
      w[4 * q] = v.x;
      w[4 * q + 1] = v.y;
      w[4 * q + 2] = v.z;
      w[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < WORDS; ++q) w[q] = p[q];
  }
}

// The dot products of one weight row (words [Gn * WORDS], scales / biases [Gn])
// with NT activation rows x[t * ld ..] held in LDS: lane l takes groups l, l + 64,
// ..; the sums are combined by the wave butterfly and returned to every lane.
template <int BITS, int G, int NT>
__device__ __forceinline__ void row_dots(const uint8_t* wrow, const uint16_t* srow, const uint16_t* brow, bool f16,
                                         int Gn, const float* x, int ld, int nt, float (&out)[NT]) {
  const int lane = threadIdx.x & 63;
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
  for (int g = lane; g < Gn; g += 64) {
    uint32_t w[G * BITS / 32];
    load_group<BITS, G>(wrow, g, w);
    const float s = scale_bits_to_f32(srow[g], f16), b = scale_bits_to_f32(brow[g], f16);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < nt) acc[t] = acc[t] + group_value<BITS, G>(w, x + t * ld + g * G, s, b);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) out[t] = wave_sum(acc[t]);
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
template <int BITS, int G, bool GROUPED>
__global__ void __launch_bounds__(THREADS) aff_gate_up_kernel(Args a) {
  extern __shared__ float xs[];   // [TB or 1][Dp] fp32
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
    if (wave == 0) {
      const int sl = route_slot(a.src, a.ws_slots, e, top_i, top_v, top_s);
      if (lane == 0) s_slot = sl;
    }
    __syncthreads();
    slot = s_slot;
  }
  const int NT = GROUPED ? nr : 1;
  // activation rows into LDS (fp32; the padding past D is zero)
  for (int t = 0; t < NT; ++t) {
    const int tok = GROUPED ? a.row_token[r0 + t] : 0;
    for (int i = tid; i < Dp; i += THREADS) xs[t * Dp + i] = i < a.D ? bf16_to_f32(a.x[(size_t)tok * a.D + i]) : 0.0f;
  }
  __syncthreads();
  const int Gn = Dp / G;
  if (slot >= 0) {
    const uint8_t* base = a.pool + (int64_t)slot * a.L.record_bytes;
    const int wb = Dp * BITS / 8;   // bytes per weight row
    // wave w: rows 4w .. 4w + 3 of W1 and W3
    for (int r = 0; r < 4; ++r) {
      const int n = row0 + 4 * wave + r;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int tq = m == 0 ? 0 : 6;
        const uint8_t* wrow = base + a.L.off[tq] + (int64_t)n * wb;
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(base + a.L.off[tq + 1]) + (int64_t)n * Gn;
        const uint16_t* brow = reinterpret_cast<const uint16_t*>(base + a.L.off[tq + 2]) + (int64_t)n * Gn;
        float v[GROUPED ? TB : 1];
        row_dots<BITS, G, GROUPED ? TB : 1>(wrow, srow, brow, a.L.f16, Gn, xs, Dp, NT, v);
        if (lane == 0)
#pragma unroll
          for (int t = 0; t < (GROUPED ? TB : 1); ++t) red[m][4 * wave + r][t] = v[t];
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
template <int BITS, int G, bool GROUPED>
__global__ void __launch_bounds__(THREADS) aff_down_kernel(Args a) {
  extern __shared__ float hs[];   // [TB][Fp] fp32
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
    __syncthreads();
    for (int t = 0; t < NT; ++t) {
      const uint16_t* hrow = a.h + (size_t)(GROUPED ? r0 + t : x) * Fp;
      for (int i = tid; i < Fp; i += THREADS) hs[t * Fp + i] = bf16_to_f32(hrow[i]);
    }
    __syncthreads();
    const int slot = slots[x];
    if (slot >= 0) {
      const uint8_t* base = a.pool + (int64_t)slot * a.L.record_bytes;
      const int wb = Fp * BITS / 8;
      for (int r = 0; r < 4; ++r) {
        const int n = row0 + 4 * wave + r;
        const uint8_t* wrow = base + a.L.off[3] + (int64_t)n * wb;
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(base + a.L.off[4]) + (int64_t)n * Gn;
        const uint16_t* brow = reinterpret_cast<const uint16_t*>(base + a.L.off[5]) + (int64_t)n * Gn;
        float v[GROUPED ? TB : 1];
        row_dots<BITS, G, GROUPED ? TB : 1>(wrow, srow, brow, a.L.f16, Gn, hs, Fp, NT, v);
        if (lane == 0)
#pragma unroll
          for (int t = 0; t < (GROUPED ? TB : 1); ++t) yv[x][4 * wave + r][t] = v[t];
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

// One thread per group of a row: w [N, row_words], scales / biases [N, groups].
template <int BITS, int G>
__global__ void __launch_bounds__(256) aff_dequant_kernel(const uint32_t* __restrict__ w,
                                                          const uint16_t* __restrict__ scales,
                                                          const uint16_t* __restrict__ biases, int N, int K,
                                                          int row_words, int groups, bool f16,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int gk = (K + G - 1) / G;
  if (i >= (int64_t)N * gk) return;
  const int64_t n = i / gk;
  const int g = (int)(i - n * gk);
  uint32_t words[G * BITS / 32];
  load_group<BITS, G>(reinterpret_cast<const uint8_t*>(w + n * row_words), g, words);
  const float s = scale_bits_to_f32(scales[n * groups + g], f16), b = scale_bits_to_f32(biases[n * groups + g], f16);
#pragma unroll
  for (int t = 0; t < G; ++t) {
    const int k = g * G + t;
    if (k < K) out[n * K + k] = s * (float)code_of<BITS>(words, t) + b;
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

template <int BITS, int G>
struct Decode {
  static int run(const Args& a, bool grouped, hipStream_t s) {
    const int Dp = (a.D + G - 1) / G * G, Fp = (a.F + G - 1) / G * G;
    const int nt = grouped ? TB : 1;
    const size_t lds_gu = (size_t)nt * Dp * 4, lds_dn = (size_t)nt * Fp * 4;
    const void* kgu = grouped ? reinterpret_cast<const void*>(aff_gate_up_kernel<BITS, G, true>)
                              : reinterpret_cast<const void*>(aff_gate_up_kernel<BITS, G, false>);
    const void* kdn = grouped ? reinterpret_cast<const void*>(aff_down_kernel<BITS, G, true>)
                              : reinterpret_cast<const void*>(aff_down_kernel<BITS, G, false>);
    if (hipFuncSetAttribute(kgu, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_gu) != hipSuccess ||
        hipFuncSetAttribute(kdn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_dn) != hipSuccess)
      return fail(CACHALOT_EHIP, "affine: cannot grant %zu / %zu bytes of LDS", lds_gu, lds_dn);
    if (grouped) {
      hipLaunchKernelGGL((aff_gate_up_kernel<BITS, G, true>), dim3((unsigned)(a.max_tiles * (a.F / 16))),
                         dim3(THREADS), lds_gu, s, a);
      if (int rc = check_launch("aff_gate_up_kernel")) return rc;
      hipLaunchKernelGGL((aff_down_kernel<BITS, G, true>), dim3((unsigned)(a.D / 16), (unsigned)a.max_tiles),
                         dim3(THREADS), lds_dn, s, a);
      return check_launch("aff_down_kernel");
    }
    hipLaunchKernelGGL((aff_gate_up_kernel<BITS, G, false>), dim3((unsigned)(a.k * (a.F / 16))), dim3(THREADS),
                       lds_gu, s, a);
    if (int rc = check_launch("aff_gate_up_kernel")) return rc;
    hipLaunchKernelGGL((aff_down_kernel<BITS, G, false>), dim3((unsigned)(a.D / 16)), dim3(THREADS), lds_dn, s, a);
    return check_launch("aff_down_kernel");
  }
};

template <int BITS, int G>
struct Dequant {
  static int run(const uint32_t* w, const uint16_t* sc, const uint16_t* bi, int N, int K, int row_words, int groups,
                 bool f16, float* out, hipStream_t s) {
    const int64_t total = (int64_t)N * ((K + G - 1) / G);
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

int decode(const uint16_t* x, const uint8_t* pool, const cachalot_expert_layout* layout, ExpertSource src,
           const RouterCall* router, int D, int F, int k, int bits, int group, float limit, const uint16_t* addend,
           float* routed, uint16_t* out, void* workspace, size_t workspace_bytes, hipStream_t s) {
  CACHALOT_REQUIRE(pool && layout && src.slot_table && x, "moe_decode_affine: null pointer");
  CACHALOT_REQUIRE(routed || out, "moe_decode_affine: no output requested");
  CACHALOT_REQUIRE(k >= 1 && k <= KMAX, "moe_decode_affine: k=%d outside 1..%d", k, KMAX);
  CACHALOT_REQUIRE(src.E >= 1 && src.E <= 1024, "moe_decode_affine: E=%d outside 1..1024", src.E);
  if (int rc = check_shape("moe_decode_affine", D, F, bits, group)) return rc;
  const WsOffsets wo = ws_offsets(hidden_bytes(k, F));
  if (workspace == nullptr || workspace_bytes < wo.total)
    return fail(CACHALOT_ESPACE, "moe_decode_affine: workspace %zu < %zu bytes", workspace_bytes, wo.total);
  Args a{};
  static const int used[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
  if (int rc = make_layout(layout, 9, used, a.L, "moe_decode_affine")) return rc;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
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
  return decode::ws_offsets(aff::hidden_bytes(k, F)).total;
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

extern "C" size_t cachalot_grouped_experts_affine_workspace_bytes(int T, int k, int E, int F) {
  if (T <= 0 || k <= 0 || E <= 0 || F <= 0) return 0;
  return aff::align256((size_t)(E + 1) * 4) + aff::hidden_bytes(T * k, F);
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
  const size_t need = cachalot_grouped_experts_affine_workspace_bytes(T, k, E, F);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CACHALOT_ESPACE, "grouped_experts_affine: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
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
