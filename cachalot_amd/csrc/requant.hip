// FP4 (E2M1 + E8M0 block-32) weights -> affine codes in MLX's layout with the
// fits of the reference's bank tool, on the GPU: benchmarks/quant_affine.py
// _quantize :113-116, _error :119-123, group_weights :126-135, fit_minmax
// :138-149, SHRINKS :155, fit_search :158-186, _lsq_step :207-228, refine_lsq
// :231-245, fit_search_lsq :255-261, SHRINKS_WIDE :281, fit_search_wide_lsq
// :284-287, quantize_affine :303-329; the fit names of build_affine_bank.py:74-75.
// Widths 2, 3 or 4 bits (L = 2^bits - 1 levels), groups of 32, 64 or 128, each
// fit optionally weighted per column by activation importance.
//
// One thread per group of a weight row: the group's FP4 values are decoded
// exactly to fp32 by the hardware converter, then
//   lo, hi, mid = (lo + hi) / 2; the min/max fit is scale = max((hi - lo) / L,
//   1e-8), bias = lo;
//   the grid fits try every shrunk range (s_lo, s_hi) over the 5 (or, wide, 9)
//   shrink factors, (1, 1) skipped, in order, and take one when its error is
//   strictly smaller; error = sum over the group in index order of
//   a (scale q + bias - w)^2, q = clip(rint((w - bias) / scale), 0, L), a the
//   column's importance (1 unweighted);
//   the LSQ fits round that pair to the storage type and run 4 assign-and-refit
//   steps: the (weighted) least-squares line through (q, w) from sums in index
//   order, rounded to the storage type; the previous pair is kept where
//   |den| < 1e-12 or the new pair is not a positive finite scale and a finite
//   bias; the best iterate (strictly smaller error) is the fit;
// then scale and bias are rounded (RNE) to the bank's storage type, bf16 or
// fp16, the codes recomputed against them (an fp16 scale that rounds to zero,
// a constant group, gives code 0) and packed as the row's little-endian bit
// stream (16, 32/3 or 8 codes per word; 3-bit codes straddle words).  Every
// operation is a single fp32 operation in the written order (the library is
// built without contraction), so the result equals a float32 evaluation in the
// same order bit for bit.  K not a multiple of the group (w2 at d_ff = 2880,
// g128): the last group fits its real elements only and its padding codes are 0.
#include "common.h"

namespace cachalot {
namespace requant {

constexpr int LSQ_ITERS = 4;
__constant__ float kShrinks[5] = {1.0f, 0.925f, 0.85f, 0.775f, 0.7f};
__constant__ float kShrinksWide[9] = {1.0f, 0.925f, 0.85f, 0.775f, 0.7f, 0.625f, 0.55f, 0.475f, 0.4f};

struct Args {
  const uint8_t* w;          // [N, K/2] packed E2M1, low nibble first
  const uint8_t* s;          // [N, K/32] E8M0
  int N, K;
  uint32_t* q;               // [N, Kp * bits / 32] codes
  uint16_t* scales;          // [N, Kp / group] bf16 or fp16 (f16)
  uint16_t* biases;          // [N, Kp / group] bf16 or fp16
  const float* importance;   // [K] per-column weights, or null
  int fit;                   // CACHALOT_FIT_*
  bool f16;
};

__device__ __forceinline__ float level(float w, float scale, float bias, float levels) {
  return fminf(fmaxf(rintf((w - bias) / scale), 0.0f), levels);
}

__device__ __forceinline__ float store_round(float v, bool f16) {
  return f16 ? scale_bits_to_f32(f32_to_f16(v), true) : round_bf16(v);
}

// Column i's weight; `a` is the group's slice of the importance vector or null.
// Past the valid elements it is never read (the last group of a ragged row).
__device__ __forceinline__ float weight_at(const float* a, int i, int nvalid) {
  return a && i < nvalid ? a[i] : 1.0f;
}

template <int G, bool W>
__device__ __forceinline__ float group_error(const float (&w)[G], const float* a, int nvalid, float scale,
                                             float bias, float levels) {
  float err = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float d = scale * level(w[i], scale, bias, levels) + bias - w[i];
    float sq = d * d;
    if constexpr (W) sq = weight_at(a, i, nvalid) * sq;
    if (i < nvalid) err = err + sq;
  }
  return err;
}

// One assign-then-refit step.
template <int G, bool W>
__device__ __forceinline__ void lsq_step(const float (&w)[G], const float* a, int nvalid, float& scale,
                                         float& bias, float levels, bool f16) {
  float n = 0.0f, sq = 0.0f, sqq = 0.0f, sw = 0.0f, sqw = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    if (i < nvalid) {
      const float q = level(w[i], scale, bias, levels);
      const float ai = W ? weight_at(a, i, nvalid) : 1.0f;
      const float aq = ai * q;
      n = n + ai;
      sq = sq + aq;
      sqq = sqq + aq * q;
      sw = sw + ai * w[i];
      sqw = sqw + aq * w[i];
    }
  }
  const float den = n * sqq - sq * sq;
  const bool sing = fabsf(den) < 1e-12f;
  const float fs = (n * sqw - sq * sw) / (sing ? 1.0f : den);
  const float ns = store_round(fs, f16);
  const float nb = store_round((sw - fs * sq) / n, f16);
  if (!(sing || !(ns > 0.0f) || !isfinite(ns) || !isfinite(nb))) {
    scale = ns;
    bias = nb;
  }
}

template <int BITS, int G, bool W>
__global__ __launch_bounds__(256) void requant_kernel(Args p) {
  constexpr float LEVELS = (float)((1 << BITS) - 1);
  constexpr int WORDS = G * BITS / 32;
  const int NG = (p.K + G - 1) / G;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)p.N * NG) return;
  const int n = (int)(gid / NG), g = (int)(gid % NG);
  const int nvalid = min(G, p.K - g * G);
  const uint8_t* wrow = p.w + (size_t)n * (p.K / 2) + (size_t)g * (G / 2);
  const uint8_t* srow = p.s + (size_t)n * (p.K / 32) + (size_t)g * (G / 32);
  const float* a = p.importance ? p.importance + (size_t)g * G : nullptr;

  float w[G];
#pragma unroll
  for (int b = 0; b < G / 32; ++b) {           // 32-element blocks: 16 code bytes + one scale
    uint4 c = make_uint4(0, 0, 0, 0);
    float sc = 1.0f;
    if (b * 32 < nvalid) {
      c = *reinterpret_cast<const uint4*>(wrow + b * 16);
      sc = e8m0_to_f32(srow[b]);
    }
    const uint32_t words[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2_t v0 = fp4x2_to_f32x2<0>(words[j], sc);
      const float2_t v1 = fp4x2_to_f32x2<1>(words[j], sc);
      const float2_t v2 = fp4x2_to_f32x2<2>(words[j], sc);
      const float2_t v3 = fp4x2_to_f32x2<3>(words[j], sc);
      float* o = w + b * 32 + j * 8;
      o[0] = v0[0]; o[1] = v0[1]; o[2] = v1[0]; o[3] = v1[1];
      o[4] = v2[0]; o[5] = v2[1]; o[6] = v3[0]; o[7] = v3[1];
    }
  }

  float lo = INFINITY, hi = -INFINITY;
#pragma unroll
  for (int i = 0; i < G; ++i)
    if (i < nvalid) {
      lo = fminf(lo, w[i]);
      hi = fmaxf(hi, w[i]);
    }
  float best_s = fmaxf((hi - lo) / LEVELS, 1e-8f), best_b = lo;
  if (p.fit != CACHALOT_FIT_MINMAX) {
    const float mid = (lo + hi) / 2.0f;
    const bool wide = p.fit == CACHALOT_FIT_WIDE_LSQ;
    const float* shr = wide ? kShrinksWide : kShrinks;
    const int ns = wide ? 9 : 5;
    float best = group_error<G, W>(w, a, nvalid, best_s, best_b, LEVELS);
    for (int x = 0; x < ns; ++x) {
      for (int y = 0; y < ns; ++y) {
        if (x == 0 && y == 0) continue;
        const float new_lo = mid + (lo - mid) * shr[x];
        const float new_hi = mid + (hi - mid) * shr[y];
        const float s = fmaxf((new_hi - new_lo) / LEVELS, 1e-8f);
        const float err = group_error<G, W>(w, a, nvalid, s, new_lo, LEVELS);
        if (err < best) {
          best_s = s;
          best_b = new_lo;
        }
        best = fminf(err, best);
      }
    }
  }
  if (p.fit == CACHALOT_FIT_SEARCH_LSQ || p.fit == CACHALOT_FIT_WIDE_LSQ) {
    float s = store_round(best_s, p.f16), b = store_round(best_b, p.f16);
    best_s = s;
    best_b = b;
    float best = group_error<G, W>(w, a, nvalid, s, b, LEVELS);
    for (int it = 0; it < LSQ_ITERS; ++it) {
      lsq_step<G, W>(w, a, nvalid, s, b, LEVELS, p.f16);
      const float err = group_error<G, W>(w, a, nvalid, s, b, LEVELS);
      if (err < best) {
        best_s = s;
        best_b = b;
      }
      best = fminf(err, best);
    }
  }

  const uint16_t sb = p.f16 ? f32_to_f16(best_s) : f32_to_bf16(best_s);
  const uint16_t bb = p.f16 ? f32_to_f16(best_b) : f32_to_bf16(best_b);
  const float s16 = scale_bits_to_f32(sb, p.f16), b16 = scale_bits_to_f32(bb, p.f16);
  uint32_t words[WORDS];
#pragma unroll
  for (int j = 0; j < WORDS; ++j) words[j] = 0u;
#pragma unroll
  for (int k = 0; k < G; ++k) {
    const uint32_t q = k < nvalid && s16 != 0.0f ? (uint32_t)level(w[k], s16, b16, LEVELS) : 0u;
    const int bit = k * BITS, wi = bit >> 5, sh = bit & 31;
    words[wi] |= q << sh;
    if (sh + BITS > 32) words[wi + 1] |= q >> (32 - sh);
  }
  uint32_t* qdst = p.q + ((size_t)n * NG + g) * WORDS;
#pragma unroll
  for (int j = 0; j < WORDS; ++j) qdst[j] = words[j];
  p.scales[(size_t)n * NG + g] = sb;
  p.biases[(size_t)n * NG + g] = bb;
}

template <int BITS, int G>
int launch(const Args& a, hipStream_t s) {
  const long groups = (long)a.N * ((a.K + G - 1) / G);
  const dim3 grid((unsigned)((groups + 255) / 256));
  if (a.importance) hipLaunchKernelGGL((requant_kernel<BITS, G, true>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((requant_kernel<BITS, G, false>), grid, dim3(256), 0, s, a);
  return check_launch("requant_fp4_to_affine");
}

}  // namespace requant
}  // namespace cachalot

using namespace cachalot;

extern "C" int cachalot_requant_fp4_to_affine(const uint8_t* w_fp4, const uint8_t* s_fp4, int N, int K, int bits,
                                              int group, int fit, const float* importance, uint32_t* q,
                                              uint16_t* scales, uint16_t* biases, int scale_dtype,
                                              cachalot_stream_t stream) {
  CACHALOT_REQUIRE(w_fp4 && s_fp4 && q && scales && biases, "requant_fp4_to_affine: null pointer");
  CACHALOT_REQUIRE(N > 0 && K > 0 && K % 32 == 0,
                   "requant_fp4_to_affine: N=%d, K=%d (K a positive multiple of 32)", N, K);
  CACHALOT_REQUIRE(((uintptr_t)w_fp4 & 15u) == 0, "requant_fp4_to_affine: w_fp4 must be 16-byte aligned");
  CACHALOT_REQUIRE(scale_dtype == CACHALOT_SCALE_BF16 || scale_dtype == CACHALOT_SCALE_F16,
                   "requant_fp4_to_affine: scale_dtype %d (0 = bf16, 1 = fp16)", scale_dtype);
  CACHALOT_REQUIRE(fit >= CACHALOT_FIT_MINMAX && fit <= CACHALOT_FIT_WIDE_LSQ,
                   "requant_fp4_to_affine: fit %d (0 minmax, 1 search, 2 search-lsq, 3 wide-lsq)", fit);
  requant::Args a{w_fp4, s_fp4, N, K, q, scales, biases, importance, fit, scale_dtype == CACHALOT_SCALE_F16};
  const hipStream_t s = (hipStream_t)stream;
#define CACHALOT_REQUANT_WIDTH(B, G) \
  if (bits == B && group == G) return requant::launch<B, G>(a, s);
  CACHALOT_REQUANT_WIDTH(2, 32) CACHALOT_REQUANT_WIDTH(2, 64) CACHALOT_REQUANT_WIDTH(2, 128)
  CACHALOT_REQUANT_WIDTH(3, 32) CACHALOT_REQUANT_WIDTH(3, 64) CACHALOT_REQUANT_WIDTH(3, 128)
  CACHALOT_REQUANT_WIDTH(4, 32) CACHALOT_REQUANT_WIDTH(4, 64) CACHALOT_REQUANT_WIDTH(4, 128)
#undef CACHALOT_REQUANT_WIDTH
  return fail(CACHALOT_EINVAL,
              "requant_fp4_to_affine: %d-bit codes in groups of %d (bits 2, 3 or 4; group 32, 64 or 128)", bits, group);
}

extern "C" int cachalot_requant_fp4_to_q2(const uint8_t* w_fp4, const uint8_t* s_fp4, int N, int K, uint32_t* q,
                                          uint16_t* scales, uint16_t* biases, int scale_dtype,
                                          cachalot_stream_t stream) {
  return cachalot_requant_fp4_to_affine(w_fp4, s_fp4, N, K, 2, 128, CACHALOT_FIT_SEARCH, nullptr, q, scales, biases,
                                        scale_dtype, stream);
}
