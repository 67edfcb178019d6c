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
// float -> E4M3FN byte, round to nearest even, for |v| <= 448 (callers clip).
// Normal range (|v| >= 2^-6): round the fp32 significand to 3 bits by adding
// half an E4M3 ulp minus one plus the kept lsb, then rebias the exponent
// (fp32 bias 127, E4M3 bias 7: field 120 << 3 = 960).  Below 2^-6 the E4M3
// value is m * 2^-9 with m = rint(|v| * 512) in 0..8 (8 is the smallest
// normal, code 0x08, so the same m is the code).  The sign is kept for zeros.
__host__ __device__ inline uint32_t e4m3_encode(float v) {
  uint32_t bits;
  __builtin_memcpy(&bits, &v, 4);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  uint32_t code;
  if (mag < 0x3c800000u) {   // 2^-6
    float a;
    __builtin_memcpy(&a, &mag, 4);
    code = (uint32_t)__builtin_rintf(a * 512.0f);
  } else {
    code = ((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - 960u;
  }
  return code | sign;
}

// Block exponent e = ceil(log2(r)) of r = fl32(amax / 448) >= 2^-23 (a normal
// float): the unbiased exponent, plus one unless the significand is exactly 1.
__host__ __device__ inline int block_exponent(float amax) {
  const float r = amax / FP8_MAX;
  uint32_t bits;
  __builtin_memcpy(&bits, &r, 4);
  return (int)((bits >> 23) & 0xffu) - 127 + ((bits & 0x7fffffu) != 0u ? 1 : 0);
}

// 2^-e as a float (e in [-23, 126]).
__device__ __forceinline__ float pow2_neg(int e) { return __uint_as_float((uint32_t)(127 - e) << 23); }

// Quantize one 32-element block: codes (8 words, element i in byte i % 4 of
// word i / 4) and the E8M0 exponent byte.
__device__ __forceinline__ uint32_t quant_block(const float (&v)[BLOCK], uint32_t (&codes)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < BLOCK; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, MIN_AMAX);
  const int e = block_exponent(amax);
  const float inv = pow2_neg(e);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float s = fminf(fmaxf(v[4 * w + b] * inv, -FP8_MAX), FP8_MAX);
      word |= e4m3_encode(s) << (8 * b);
    }
    codes[w] = word;
  }
  return (uint32_t)(e + 127);
}

struct QuantArgs {
  const uint16_t* x;      // act_quant: x [M, K] bf16 (row stride ldx); swiglu: gu [M, 2K] bf16 (g | u)
  int ldx;
  int M, K;               // K = row length of the quantized output
  float limit;            // swiglu clamp (<= 0: none)
  uint8_t* q;             // [M, K] E4M3
  uint8_t* e;             // [M, K / 32] E8M0
};

__device__ __forceinline__ void load_bf16x32(const uint16_t* src, float (&v)[BLOCK]) {
  const uint4* p = reinterpret_cast<const uint4*>(src);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 w = p[j];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[8 * j + 2 * i] = __uint_as_float(ws[i] << 16);
      v[8 * j + 2 * i + 1] = __uint_as_float(ws[i] & 0xffff0000u);
    }
  }
}

// One thread per 32-element block.  SWIGLU: the block's h values first,
// h = bf16(silu(min(g, L)) * clip(u, -L, L)) from the bf16 g and u.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void quant_kernel(QuantArgs p) {
  const int nb = p.K / BLOCK;
  const long blk = (long)blockIdx.x * 256 + threadIdx.x;
  if (blk >= (long)p.M * nb) return;
  const int t = (int)(blk / nb), b = (int)(blk % nb);
  float v[BLOCK];
  if constexpr (SWIGLU) {
    float u[BLOCK];
    const uint16_t* row = p.x + (size_t)t * p.ldx;
    load_bf16x32(row + b * BLOCK, v);
    load_bf16x32(row + p.K + b * BLOCK, u);
#pragma unroll
    for (int i = 0; i < BLOCK; ++i) {
      float g = v[i], uu = u[i];
      if (p.limit > 0.0f) {
        uu = fminf(fmaxf(uu, -p.limit), p.limit);
        g = fminf(g, p.limit);
      }
      v[i] = round_bf16(decode::silu_f32(g) * uu);
    }
  } else {
    load_bf16x32(p.x + (size_t)t * p.ldx + b * BLOCK, v);
  }
  uint32_t codes[8];
  const uint32_t eb = quant_block(v, codes);
  uint4* dst = reinterpret_cast<uint4*>(p.q + (size_t)t * p.K + b * BLOCK);
  dst[0] = make_uint4(codes[0], codes[1], codes[2], codes[3]);
  dst[1] = make_uint4(codes[4], codes[5], codes[6], codes[7]);
  p.e[(size_t)t * nb + b] = (uint8_t)eb;
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

__device__ __forceinline__ Operand load_operand(const uint8_t* base, const uint8_t* scales, int K, int c, int kg,
                                                bool row_ok) {
  Operand o;
  const int k0 = c * CHUNK + BLOCK * kg;
  o.lo = make_uint4(0, 0, 0, 0);
  o.hi = make_uint4(0, 0, 0, 0);
  if (row_ok && k0 < K) {
    o.lo = *reinterpret_cast<const uint4*>(base + k0);
    o.hi = *reinterpret_cast<const uint4*>(base + k0 + 16);
  }
  const int blk = 4 * c + kg;
  o.s = blk < K / BLOCK ? (uint32_t)scales[blk] : E8M0_ONE;
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
  const long blocks = (long)M * (K / BLOCK);
  const dim3 grid((unsigned)((blocks + 255) / 256));
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
  if (M == 0) return CACHALOT_OK;
  return fp8::launch_quant(x, K, M, K, false, 0.0f, q, scales, (hipStream_t)stream);
}

extern "C" int cachalot_fp8_linear_quantized(const uint8_t* q, const uint8_t* q_scales, const uint8_t* w,
                                             const uint8_t* w_scales, int M, int K, int N, uint16_t* y,
                                             cachalot_stream_t stream) {
  if (int rc = fp8::check_shapes("fp8_linear_quantized", M, K, N)) return rc;
  CACHALOT_REQUIRE(q && q_scales && w && w_scales && y, "fp8_linear_quantized: null pointer");
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
  if (M == 0) return CACHALOT_OK;
  const size_t need = fp8::workspace_bytes(M, D, F);
  if (workspace_bytes < need || !workspace)
    return fail(CACHALOT_ESPACE, "shared_expert_fp8: workspace %zu bytes < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const fp8::Workspace ws = fp8::carve(workspace, M, D, F);
  if (int rc = fp8::launch_quant(x, D, M, D, false, 0.0f, ws.xq, ws.xe, s)) return rc;
  fp8::LinearArgs gu{ws.xq, ws.xe, {w1, w3}, {w1_scales, w3_scales}, M, F, D, ws.gu, 2 * F};
  if (int rc = fp8::launch_linear(gu, 2, s)) return rc;
  if (int rc = fp8::launch_quant(ws.gu, 2 * F, M, F, true, swiglu_limit, ws.hq, ws.he, s)) return rc;
  fp8::LinearArgs dn{ws.hq, ws.he, {w2, w2}, {w2_scales, w2_scales}, M, D, F, y, D};
  return fp8::launch_linear(dn, 1, s);
}
