// Shared FP8 expert and FP8 linear on the gfx950 block-scaled matrix cores.
//
// Semantics (src/cachalot/model/fp8_ref.py:28-231, fp8_linear_metal.py:30-107,
// shared_expert_metal.py:44-188, moe_prefill_batched.py:64-125):
//   act_quant, per 32-element block of a row: amax = max(max|v|, 1e-4),
//     e = ceil(log2(fl32(amax / 448))), q = E4M3(clip(v / 2^e, -448, 448)) (RNE);
//   linear: y[t, n] = bf16( sum_kb (q_t,kb . w_n,kb) 2^e[t,kb] 2^(ws[n/32,kb]-127) )
//     with fp32 accumulation;
//   shared expert: g = bf16(w1 q), u = bf16(w3 q); u = clip(u, -L, L), g = min(g, L)
//     (L > 0); h = bf16(silu(g) u); y = bf16(w2 act_quant(h)).
//
// Arithmetic: an E4M3 value times its power-of-two block scale is exact in
// bf16, so activations and weights are converted in registers (gfx950 scaled
// fp8 -> bf16 converter, block scale folded in) and multiplied on the bf16
// matrix cores (v_mfma_f32_16x16x32_bf16), whose products are exact in fp32 and
// whose accumulation is fp32: the reference's sum of per-block dot products
// times act_scale x weight_scale, up to fp32 summation order.  Activations
// travel as E4M3 bytes + E8M0 exponents (1 byte per value), weights as the
// checkpoint's bytes.  D[i][j] of a 16x16 tile is in lane j + 16 (i / 4),
// register i % 4.
//
// Launches: quant(x) -> linear(w1 | w3) -> swiglu+quant(h) -> linear(w2).
#include "common.h"
#include "decode_common.h"

namespace cachalot {
namespace fp8 {

typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int BLOCK = 32;
constexpr int CHUNK = 128;
constexpr float FP8_MAX = 448.0f;
constexpr float MIN_AMAX = 1e-4f;
constexpr uint32_t E8M0_ONE = 127u;

// ------------------------------------------------------------ act_quant ---
// Block exponent e = ceil(log2(r)) of r = fl32(amax / 448) >= 2^-23 (a normal
// float): the unbiased exponent, plus one unless the significand is exactly 1.
__device__ __forceinline__ int block_exponent(float amax) {
  const uint32_t bits = __float_as_uint(amax / FP8_MAX);
  return (int)((bits >> 23) & 0xffu) - 127 + ((bits & 0x7fffffu) != 0u ? 1 : 0);
}

// 2^-e as a float (e in [-23, 126]).
__device__ __forceinline__ float pow2_neg(int e) { return __uint_as_float((uint32_t)(127 - e) << 23); }

__device__ __forceinline__ float clip448(float v) { return fminf(fmaxf(v, -FP8_MAX), FP8_MAX); }

// One quarter (8 consecutive values) of a 32-element block whose four quarters
// sit in an aligned group of 4 lanes (quarter q in lane 4 g + q): the block's
// exponent (amax over the 4 lanes by two quad swaps) and this quarter's E4M3
// codes, element i in byte i % 4 of word i / 4, converted by the hardware
// round-to-nearest-even fp32 -> E4M3 converter after the exact power-of-two
// scaling and the clip.  Every lane of the wave must execute it.
__device__ __forceinline__ uint2 quant_quarter(const float (&v)[8], int& e) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __uint_as_float(xor1_u32(__float_as_uint(amax))));
  amax = fmaxf(amax, __uint_as_float(xor2_u32(__float_as_uint(amax))));
  e = block_exponent(fmaxf(amax, MIN_AMAX));
  const float inv = pow2_neg(e);
  uint2 w;
  int t = __builtin_amdgcn_cvt_pk_fp8_f32(clip448(v[0] * inv), clip448(v[1] * inv), 0, false);
  w.x = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clip448(v[2] * inv), clip448(v[3] * inv), t, true);
  t = __builtin_amdgcn_cvt_pk_fp8_f32(clip448(v[4] * inv), clip448(v[5] * inv), 0, false);
  w.y = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clip448(v[6] * inv), clip448(v[7] * inv), t, true);
  return w;
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& w, float (&v)[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(ws[i] << 16);
    v[2 * i + 1] = __uint_as_float(ws[i] & 0xffff0000u);
  }
}

// h = bf16(silu(min(g, L)) * clip(u, -L, L)) from bf16 g and u (L <= 0: no clamp).
__device__ __forceinline__ float swiglu_h(float g, float u, float limit) {
  if (limit > 0.0f) {
    u = fminf(fmaxf(u, -limit), limit);
    g = fminf(g, limit);
  }
  return round_bf16(decode::silu_f32(g) * u);
}

struct QuantArgs {
  const uint16_t* x;      // act_quant: x [M, K] bf16 (row stride ldx); swiglu: gu [M, 2K] bf16 (g | u)
  int ldx;
  int M, K;               // K = row length of the quantized output
  float limit;            // swiglu clamp (<= 0: none)
  uint8_t* q;             // [M, K] E4M3
  uint8_t* e;             // [M, K / 32] E8M0
};

// Four lanes per 32-element block, 8 values (one 16-byte load) each.  SWIGLU:
// the values are h = swiglu(g, u) from the bf16 g | u rows.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void quant_kernel(QuantArgs p) {
  const int nq = p.K / 8;                                   // quarters per row
  const long qi = (long)blockIdx.x * 256 + threadIdx.x;
  const bool ok = qi < (long)p.M * nq;
  const int t = ok ? (int)(qi / nq) : 0, k8 = ok ? (int)(qi % nq) * 8 : 0;
  const uint16_t* row = p.x + (size_t)t * p.ldx;
  float v[8];
  if (ok) {
    unpack_bf16x8(*reinterpret_cast<const uint4*>(row + k8), v);
    if constexpr (SWIGLU) {
      float u[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(row + p.K + k8), u);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = swiglu_h(v[i], u[i], p.limit);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  int e;
  const uint2 w = quant_quarter(v, e);
  if (!ok) return;
  *reinterpret_cast<uint2*>(p.q + (size_t)t * p.K + k8) = w;
  if ((k8 & 31) == 0) p.e[(size_t)t * (p.K / BLOCK) + k8 / BLOCK] = (uint8_t)(e + 127);
}

// --------------------------------------------------------------- linear ---
struct LinearArgs {
  const uint8_t* a;          // [M, K] E4M3 activations
  const uint8_t* ae;         // [M, K / 32] E8M0
  const uint8_t* w[2];       // per matrix [N, K] E4M3 weights
  const uint8_t* ws[2];      // per matrix [ceil(N / 32), K / 32] E8M0
  int M, N, K;               // N rows per matrix
  uint16_t* out;             // bf16: out[t * ldo + mat * N + n]
  int ldo;
};

// A lane's share of one 128-element chunk of a row: K [128 c + 32 kg, +32) of
// an E4M3 row (zeros past K or for an invalid row) and the E8M0 scale of that
// 32-element block (1.0 past K).
struct Operand {
  uint4 lo, hi;
  uint32_t s;
};

// Branch-free: out-of-range lanes load from the row start and are zeroed after,
// so every load is issued unconditionally and the compiler can wait for exactly
// the loads a use needs (loads under a branch make it wait for all of them).
__device__ __forceinline__ Operand load_operand(const uint8_t* base, const uint8_t* scales, int K, int c, int kg,
                                                bool row_ok) {
  Operand o;
  const int k0 = c * CHUNK + BLOCK * kg;
  const bool ok = row_ok && k0 < K;
  const int kk = ok ? k0 : 0, blk = ok ? 4 * c + kg : 0;
  const uint4 lo = *reinterpret_cast<const uint4*>(base + kk);
  const uint4 hi = *reinterpret_cast<const uint4*>(base + kk + 16);
  const uint32_t sc = scales[blk];
  const uint4 z = make_uint4(0, 0, 0, 0);
  o.lo = ok ? lo : z;
  o.hi = ok ? hi : z;
  o.s = ok ? sc : E8M0_ONE;
  return o;
}

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;

// Eight E4M3 values (two words) times their block scale, as bf16 (exact: 4
// significant bits and a power-of-two factor), by the gfx950 scaled converter.
__device__ __forceinline__ bf16x8_t to_bf16x8(uint32_t w0, uint32_t w1, float scale) {
  uint4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true));
  return __builtin_bit_cast(bf16x8_t, r);
}

// The eight values of step j (0..3) of an operand: bytes [8 j, 8 j + 8) of its 32.
__device__ __forceinline__ bf16x8_t step_values(const Operand& o, int j, float scale) {
  const uint32_t w[8] = {o.lo.x, o.lo.y, o.lo.z, o.lo.w, o.hi.x, o.hi.y, o.hi.z, o.hi.w};
  return to_bf16x8(w[2 * j], w[2 * j + 1], scale);
}

// Products of scaled E4M3 values are exact in fp32 and the bf16 matrix cores
// accumulate them in fp32, the reference's arithmetic.  (The fp8 matrix-core
// instructions were measured to align products to the largest one and drop
// bits about 2^-19 below it, far from fp32 accumulation on wide-range data.)
__device__ __forceinline__ f32x4_t mfma_bf16(const bf16x8_t& a, const bf16x8_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroup = 4 waves = 16 MT tokens x 16 RT rows of one matrix; the waves split
// the K chunks (wave w: chunks w, w + 4, ..), loading PF chunks at a time, and
// their partial tiles are summed in LDS in wave order.  A chunk is four
// 16x16x32 steps; in step j lane (c, kg) carries K 128 chunk + 32 kg + 8 j + [0, 8)
// of its token row (A) and weight row (B).
template <int MT, int RT, int PF>
__global__ __launch_bounds__(256) void linear_kernel(LinearArgs p) {
  __shared__ float red[4][MT * RT][64][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, kg = lane >> 4;
  const int row0 = blockIdx.x * 16 * RT;              // row over the stacked matrices
  const int mat = row0 / p.N, n0 = row0 - mat * p.N;
  const int t0 = blockIdx.y * 16 * MT;
  const int nch = (p.K + CHUNK - 1) / CHUNK, nkb = p.K / BLOCK;
  const uint8_t* w = p.w[mat];
  const uint8_t* ws = p.ws[mat];

  const uint8_t* brow[RT];
  const uint8_t* bsc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int n = n0 + 16 * r + c16;
    brow[r] = w + (size_t)n * p.K;
    bsc[r] = ws + (size_t)((n0 + 16 * r) / 32) * nkb;
  }
  const uint8_t* arow[MT];
  const uint8_t* asc[MT];
  bool aok[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int t = t0 + 16 * m + c16;
    aok[m] = t < p.M;
    arow[m] = p.a + (size_t)(aok[m] ? t : 0) * p.K;
    asc[m] = p.ae + (size_t)(aok[m] ? t : 0) * nkb;
  }

  f32x4_t acc[MT][RT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[m][r] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int c0 = wave; c0 < nch; c0 += 4 * PF) {
    Operand B[PF][RT], A[PF][MT];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = c0 + 4 * i;
      const bool ok = c < nch;
#pragma unroll
      for (int r = 0; r < RT; ++r) B[i][r] = load_operand(brow[r], bsc[r], ok ? p.K : 0, c, kg, true);
#pragma unroll
      for (int m = 0; m < MT; ++m) A[i][m] = load_operand(arow[m], asc[m], ok ? p.K : 0, c, kg, aok[m]);
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (c0 + 4 * i >= nch) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8_t bv[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) bv[r] = step_values(B[i][r], j, e8m0_to_f32(B[i][r].s));
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const bf16x8_t av = step_values(A[i][m], j, e8m0_to_f32(A[i][m].s));
#pragma unroll
          for (int r = 0; r < RT; ++r) acc[m][r] = mfma_bf16(av, bv[r], acc[m][r]);
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][m * RT + r][lane][j] = acc[m][r][j];
  __syncthreads();

  // Thread -> (token i, row j) of each 16 x 16 tile; D[i][j] is lane j + 16 (i / 4), register i % 4.
  const int j = threadIdx.x & 15, i = threadIdx.x >> 4;
  const int dl = j + 16 * (i >> 2), dr = i & 3;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int t = t0 + 16 * m + i;
    if (t >= p.M) continue;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int tile = m * RT + r;
      const float s = ((red[0][tile][dl][dr] + red[1][tile][dl][dr]) + red[2][tile][dl][dr]) + red[3][tile][dl][dr];
      p.out[(size_t)t * p.ldo + mat * p.N + n0 + 16 * r + j] = f32_to_bf16(s);
    }
  }
}

// ---------------------------------------------------------- decode GEMV ---
// Few tokens (M <= DEC_MT per workgroup tile): the activation rows are
// quantized by the workgroup itself into LDS (E4M3 codes + E8M0 exponents, the
// act_quant above), so a decode call is two launches:
//   gate/up (PAIRED): a 16-column tile = 8 rows of w1 and the same 8 rows of w3;
//     the epilogue forms h = bf16(silu(min(g, L)) * clip(u, -L, L)) from the
//     bf16-rounded g and u of each row and writes h [M, F] bf16;
//   down: 16 rows of w2 over act_quant(h), y [M, D] bf16.
// The waves split the K chunks; a wave's first PF chunks of weights are
// requested before the activation rows are quantized, so the HBM stream starts
// at once (the activation loads are issued first, so waiting for them leaves
// the weight loads in flight).
constexpr int DEC_MT = 4;
constexpr int DEC_MAX_K = 5120;
#ifndef CACHALOT_DEC_WAVES
#define CACHALOT_DEC_WAVES 16
#endif
constexpr int DEC_WAVES = CACHALOT_DEC_WAVES;      // waves per workgroup (they split K)
constexpr int DEC_PF = 32 / DEC_WAVES;             // chunks of weights in flight per wave

struct DecodeArgs {
  const uint16_t* a;         // bf16 activation rows [M, K], row stride lda
  int lda;
  const uint8_t* w[2];       // w1, w3 (PAIRED) or w2
  const uint8_t* ws[2];
  int M, N, K;               // N = rows per matrix
  float limit;
  uint16_t* out;             // PAIRED: h [M, N]; else y [M, N]; row stride ldo
  int ldo;
};

__host__ __device__ inline int dec_stride(int K) { return K + 16; }
__host__ __device__ inline int dec_lds_bytes(int K, int waves) {
  const int codes = DEC_MT * dec_stride(K), scales = DEC_MT * (K / BLOCK);
  return ((codes + scales + 15) & ~15) + waves * 64 * 4 * 4;
}

template <bool PAIRED, int WAVES, int PF>
__global__ __launch_bounds__(WAVES * 64) void decode_kernel(DecodeArgs p) {
  constexpr int NT = WAVES * 64;
  constexpr int XP = (DEC_MT * DEC_MAX_K / 8 + NT - 1) / NT;   // activation quarters per thread
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, kg = lane >> 4;
  const int K = p.K, nkb = K / BLOCK, nch = (K + CHUNK - 1) / CHUNK, stride = dec_stride(K);
  const int t0 = blockIdx.y * DEC_MT, mt = min(DEC_MT, p.M - t0);
  uint8_t* codes = lds;
  uint8_t* scl = lds + DEC_MT * stride;
  float* red = reinterpret_cast<float*>(lds + ((DEC_MT * stride + DEC_MT * nkb + 15) & ~15));

  // 1. the activation quarters this thread quantizes (loads first in program order)
  const int nq = K / 8, total = mt * nq;
  uint4 xv[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int q = min(threadIdx.x + NT * i, total - 1);     // unconditional load; extra lanes are unused
    const int r = q / nq, k8 = (q - r * nq) * 8;
    xv[i] = *reinterpret_cast<const uint4*>(p.a + (size_t)(t0 + r) * p.lda + k8);
  }
  __builtin_amdgcn_sched_barrier(0);   // keep the activation loads ahead of the weight loads

  // 2. this wave's first PF chunks of weights
  int mat, n;
  if constexpr (PAIRED) {
    mat = c16 >> 3;
    n = blockIdx.x * 8 + (c16 & 7);
  } else {
    mat = 0;
    n = blockIdx.x * 16 + c16;
  }
  // (select, not index: a lane-dependent index into the argument block would be a
  // vector memory load, ordered behind the activation loads above)
  const uint8_t* brow = (mat ? p.w[1] : p.w[0]) + (size_t)n * K;
  const uint8_t* bsc = (mat ? p.ws[1] : p.ws[0]) + (size_t)(n / 32) * nkb;
  Operand B[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    const int c = wave + WAVES * i;
    B[i] = load_operand(brow, bsc, c < nch ? K : 0, c, kg, true);
  }

  // 3. quantize the activation rows into LDS
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    if (NT * i >= total) break;                        // uniform
    const int q = threadIdx.x + NT * i;
    float v[8];
    unpack_bf16x8(q < total ? xv[i] : make_uint4(0, 0, 0, 0), v);
    int e;
    const uint2 w = quant_quarter(v, e);
    if (q < total) {
      const int r = q / nq, k8 = (q - r * nq) * 8;
      *reinterpret_cast<uint2*>(codes + r * stride + k8) = w;
      if ((k8 & 31) == 0) scl[r * nkb + k8 / BLOCK] = (uint8_t)(e + 127);
    }
  }
  lds_sync();

  // 4. chunks: A from LDS (rows >= mt are zero), B from registers
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = wave;; c0 += WAVES * PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = c0 + WAVES * i;
      if (c >= nch) break;
      const int k0 = c * CHUNK + BLOCK * kg;
      Operand A;
      A.lo = make_uint4(0, 0, 0, 0);
      A.hi = make_uint4(0, 0, 0, 0);
      A.s = E8M0_ONE;
      if (c16 < mt && k0 < K) {
        A.lo = *reinterpret_cast<const uint4*>(codes + c16 * stride + k0);
        A.hi = *reinterpret_cast<const uint4*>(codes + c16 * stride + k0 + 16);
        A.s = scl[c16 * nkb + 4 * c + kg];
      }
      const float sa = e8m0_to_f32(A.s), sb = e8m0_to_f32(B[i].s);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma_bf16(step_values(A, j, sa), step_values(B[i], j, sb), acc);
    }
    if (c0 + WAVES * PF >= nch) break;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = c0 + WAVES * PF + WAVES * i;
      B[i] = load_operand(brow, bsc, c < nch ? K : 0, c, kg, true);
    }
  }

  // 5. sum the waves' tiles in wave order; D[i][j] is lane j + 16 (i / 4), register i % 4
#pragma unroll
  for (int j = 0; j < 4; ++j) red[(wave * 64 + lane) * 4 + j] = acc[j];
  __syncthreads();
  const int j = threadIdx.x & 15, i = threadIdx.x >> 4;
  if (i >= mt) return;
  auto total_of = [&](int col) {
    const int idx = ((col + 16 * (i >> 2)) * 4) + (i & 3);
    float t = red[idx];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[256 * w + idx];
    return t;
  };
  if constexpr (PAIRED) {
    if (j >= 8) return;
    const float g = round_bf16(total_of(j)), u = round_bf16(total_of(j + 8));
    p.out[(size_t)(t0 + i) * p.ldo + blockIdx.x * 8 + j] = f32_to_bf16(swiglu_h(g, u, p.limit));
  } else {
    p.out[(size_t)(t0 + i) * p.ldo + blockIdx.x * 16 + j] = f32_to_bf16(total_of(j));
  }
}

// ------------------------------------------------------------------ host ---
inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct Workspace {
  uint8_t *xq, *xe, *hq, *he;
  uint16_t* gu;
};

inline size_t workspace_bytes(int M, int D, int F) {
  return align256((size_t)M * D) + align256((size_t)M * (D / BLOCK)) + align256((size_t)M * 2 * F * 2) +
         align256((size_t)M * F) + align256((size_t)M * (F / BLOCK));
}

inline Workspace carve(void* base, int M, int D, int F) {
  uint8_t* p = static_cast<uint8_t*>(base);
  Workspace w;
  w.xq = p; p += align256((size_t)M * D);
  w.xe = p; p += align256((size_t)M * (D / BLOCK));
  w.gu = reinterpret_cast<uint16_t*>(p); p += align256((size_t)M * 2 * F * 2);
  w.hq = p; p += align256((size_t)M * F);
  w.he = p;
  return w;
}

int launch_quant(const uint16_t* x, int ldx, int M, int K, bool swiglu, float limit, uint8_t* q, uint8_t* e,
                 hipStream_t s) {
  QuantArgs a{x, ldx, M, K, limit, q, e};
  const long quarters = (long)M * (K / 8);
  const dim3 grid((unsigned)((quarters + 255) / 256));
  if (swiglu)
    hipLaunchKernelGGL(quant_kernel<true>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(quant_kernel<false>, grid, dim3(256), 0, s, a);
  return check_launch("fp8 quant");
}

// Tile choice: token-tiled GEMV (one 16-token tile per workgroup, 8 chunks of
// every wave in flight) for decode-sized M; 64 x 64 tiles for many tokens.
int launch_linear(const LinearArgs& a, int nmat, hipStream_t s) {
  if (a.M > 64 && a.N % 64 == 0) {
    const dim3 grid((unsigned)(nmat * a.N / 64), (unsigned)((a.M + 63) / 64));
    hipLaunchKernelGGL((linear_kernel<4, 4, 1>), grid, dim3(256), 0, s, a);
  } else {
    const dim3 grid((unsigned)(nmat * a.N / 16), (unsigned)((a.M + 15) / 16));
    hipLaunchKernelGGL((linear_kernel<1, 1, 8>), grid, dim3(256), 0, s, a);
  }
  return check_launch("fp8 linear");
}

// Decode (M <= DEC_MT): gate/up + SwiGLU -> h [M, F] bf16 (in the gu region), down -> y.
int launch_decode(const uint16_t* x, const uint8_t* w1, const uint8_t* s1, const uint8_t* w3, const uint8_t* s3,
                  const uint8_t* w2, const uint8_t* s2, int M, int D, int F, float limit, uint16_t* h, uint16_t* y,
                  hipStream_t s) {
  DecodeArgs gu{x, D, {w1, w3}, {s1, s3}, M, F, D, limit, h, F};
  const dim3 grid_gu((unsigned)(F / 8), (unsigned)((M + DEC_MT - 1) / DEC_MT));
  hipLaunchKernelGGL((decode_kernel<true, DEC_WAVES, DEC_PF>), grid_gu, dim3(64 * DEC_WAVES), dec_lds_bytes(D, DEC_WAVES),
                     s, gu);
  if (int rc = check_launch("fp8 decode gate/up")) return rc;
  DecodeArgs dn{h, F, {w2, w2}, {s2, s2}, M, D, F, limit, y, D};
  const dim3 grid_dn((unsigned)(D / 16), (unsigned)((M + DEC_MT - 1) / DEC_MT));
  hipLaunchKernelGGL((decode_kernel<false, DEC_WAVES, DEC_PF>), grid_dn, dim3(64 * DEC_WAVES),
                     dec_lds_bytes(F, DEC_WAVES), s, dn);
  return check_launch("fp8 decode down");
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_shapes(const char* who, int M, int K, int N) {
  CACHALOT_REQUIRE(M >= 0, "%s: M=%d must be >= 0", who, M);
  CACHALOT_REQUIRE(K > 0 && K % BLOCK == 0, "%s: K=%d must be a positive multiple of %d", who, K, BLOCK);
  CACHALOT_REQUIRE(N > 0 && N % 16 == 0, "%s: N=%d must be a positive multiple of 16", who, N);
  return CACHALOT_OK;
}

}  // namespace fp8
}  // namespace cachalot

using namespace cachalot;

extern "C" int cachalot_fp8_act_quant(const uint16_t* x, int M, int K, uint8_t* q, uint8_t* scales,
                                      cachalot_stream_t stream) {
  CACHALOT_REQUIRE(M >= 0, "fp8_act_quant: M=%d must be >= 0", M);
  CACHALOT_REQUIRE(K > 0 && K % fp8::BLOCK == 0, "fp8_act_quant: K=%d must be a positive multiple of 32", K);
  CACHALOT_REQUIRE(x && q && scales, "fp8_act_quant: null pointer");
  CACHALOT_REQUIRE(fp8::aligned16(x) && fp8::aligned16(q), "fp8_act_quant: x and q must be 16-byte aligned");
  if (M == 0) return CACHALOT_OK;
  return fp8::launch_quant(x, K, M, K, false, 0.0f, q, scales, (hipStream_t)stream);
}

extern "C" int cachalot_fp8_linear_quantized(const uint8_t* q, const uint8_t* q_scales, const uint8_t* w,
                                             const uint8_t* w_scales, int M, int K, int N, uint16_t* y,
                                             cachalot_stream_t stream) {
  if (int rc = fp8::check_shapes("fp8_linear_quantized", M, K, N)) return rc;
  CACHALOT_REQUIRE(q && q_scales && w && w_scales && y, "fp8_linear_quantized: null pointer");
  CACHALOT_REQUIRE(fp8::aligned16(q) && fp8::aligned16(w), "fp8_linear_quantized: q and w must be 16-byte aligned");
  if (M == 0) return CACHALOT_OK;
  fp8::LinearArgs a{q, q_scales, {w, w}, {w_scales, w_scales}, M, N, K, y, N};
  return fp8::launch_linear(a, 1, (hipStream_t)stream);
}

extern "C" size_t cachalot_shared_expert_fp8_workspace_bytes(int M, int D, int F) {
  if (M <= 0 || D <= 0 || F <= 0) return 0;
  return fp8::workspace_bytes(M, D, F);
}

extern "C" int cachalot_shared_expert_fp8(const uint16_t* x, const uint8_t* w1, const uint8_t* w1_scales,
                                          const uint8_t* w3, const uint8_t* w3_scales, const uint8_t* w2,
                                          const uint8_t* w2_scales, int M, int D, int F, float swiglu_limit,
                                          uint16_t* y, void* workspace, size_t workspace_bytes,
                                          cachalot_stream_t stream) {
  if (int rc = fp8::check_shapes("shared_expert_fp8 (w1/w3)", M, D, F)) return rc;
  if (int rc = fp8::check_shapes("shared_expert_fp8 (w2)", M, F, D)) return rc;
  CACHALOT_REQUIRE(x && w1 && w1_scales && w3 && w3_scales && w2 && w2_scales && y,
                   "shared_expert_fp8: null pointer");
  CACHALOT_REQUIRE(fp8::aligned16(x) && fp8::aligned16(w1) && fp8::aligned16(w3) && fp8::aligned16(w2) &&
                       fp8::aligned16(workspace),
                   "shared_expert_fp8: x, the weights and the workspace must be 16-byte aligned");
  if (M == 0) return CACHALOT_OK;
  const size_t need = fp8::workspace_bytes(M, D, F);
  if (workspace_bytes < need || !workspace)
    return fail(CACHALOT_ESPACE, "shared_expert_fp8: workspace %zu bytes < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const fp8::Workspace ws = fp8::carve(workspace, M, D, F);
  if (M <= fp8::DEC_MT && D <= fp8::DEC_MAX_K && F <= fp8::DEC_MAX_K && F % 8 == 0)
    return fp8::launch_decode(x, w1, w1_scales, w3, w3_scales, w2, w2_scales, M, D, F, swiglu_limit, ws.gu, y, s);
  if (int rc = fp8::launch_quant(x, D, M, D, false, 0.0f, ws.xq, ws.xe, s)) return rc;
  fp8::LinearArgs gu{ws.xq, ws.xe, {w1, w3}, {w1_scales, w3_scales}, M, F, D, ws.gu, 2 * F};
  if (int rc = fp8::launch_linear(gu, 2, s)) return rc;
  if (int rc = fp8::launch_quant(ws.gu, 2 * F, M, F, true, swiglu_limit, ws.hq, ws.he, s)) return rc;
  fp8::LinearArgs dn{ws.hq, ws.he, {w2, w2}, {w2_scales, w2_scales}, M, D, F, y, D};
  return fp8::launch_linear(dn, 1, s);
}
