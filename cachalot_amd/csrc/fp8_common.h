// FP8 (E4M3 values, E8M0 block-32 scales) building blocks of the shared expert:
// act_quant, operand loads and conversion for the bf16 matrix cores, and the
// decode tile that the shared expert's own launches and the routed decode
// launches that carry it (decode_q2_mx.hip) both run.
//
// Semantics: src/cachalot/model/fp8_ref.py:28-231 (act_quant, the block-scaled
// linear), shared_expert_metal.py:44-188 (the expert's casts).
#pragma once
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
// ---------------------------------------------------------- decode tile ---
// Few tokens (M <= DEC_MT): a 16-column tile of one product, the activation rows
// quantized into LDS by the workgroup itself (act_quant), the weights streamed
// into registers.  PAIRED: 8 rows of w1 and the same 8 rows of w3 (columns 0-7,
// 8-15); else 16 rows of one matrix.
//
// The K chunks (128 elements) are dealt to DEC_VW = 16 virtual waves -- virtual
// wave v takes chunks v, v + 16, v + 32, .. in that order, into its own
// accumulator -- and the 16 partial tiles are summed in v order.  RW real waves
// run them (wave w: v = w, w + RW, ..), so the summation order, and with it every
// output bit, is the same whatever RW a launch uses: the shared expert's own
// launches (RW = 16) and the routed decode launches that carry the shared
// expert (RW = 4 in gate/up, 12 in down) agree bit for bit.
constexpr int DEC_VW = 16;
constexpr int DEC_MT = 4;
constexpr int DEC_MAX_K = 5120;

struct DecodeArgs {
  const uint16_t* a;         // bf16 activation rows [M, K], row stride lda
  int lda;
  const uint8_t* w[2];       // w1, w3 (PAIRED) or w2 (both entries)
  const uint8_t* ws[2];
  int M, N, K;               // N = rows per matrix
  float limit;
  uint16_t* out;             // PAIRED: h [M, N]; else y [M, N]; row stride ldo
  int ldo;
};

__host__ __device__ constexpr int dec_stride(int K) { return K + 16; }
// LDS of a tile with up to MT tokens: codes [MT][K + 16], exponents [MT][K / 32],
// then the partial tiles red [16 virtual waves][16 lanes][4] (tokens < 4 sit in
// lanes 0-15 of an accumulator, token t in register t).
__host__ __device__ constexpr int dec_red_offset(int MT, int K) { return (MT * dec_stride(K) + MT * (K / BLOCK) + 15) & ~15; }
__host__ __device__ constexpr int dec_tile_lds(int MT, int K) { return dec_red_offset(MT, K) + DEC_VW * 16 * 4 * 4; }

template <int MT, int NT>
struct DecAct {
  uint4 v[(MT * DEC_MAX_K / 8 + NT - 1) / NT];   // activation quarters of this thread
};

// 1. the activation quarters of tokens t0 .. t0 + mt - 1 (unconditional loads;
//    extra lanes re-read the last quarter and are unused)
template <int MT, int NT>
__device__ __forceinline__ void dec_act_load(const DecodeArgs& p, int t0, int mt, int tid, DecAct<MT, NT>& xa) {
  const int nq = p.K / 8, total = mt * nq;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(xa.v) / sizeof(xa.v[0])); ++i) {
    const int q = min(tid + NT * i, total - 1);
    const int r = q / nq, k8 = (q - r * nq) * 8;
    xa.v[i] = *reinterpret_cast<const uint4*>(p.a + (size_t)(t0 + r) * p.lda + k8);
  }
}

// 2. act_quant of the loaded rows into LDS (every thread of the workgroup calls it)
template <int MT, int NT>
__device__ __forceinline__ void dec_act_quant(const DecodeArgs& p, int mt, int tid, const DecAct<MT, NT>& xa,
                                              uint8_t* lds) {
  const int K = p.K, nq = K / 8, total = mt * nq, nkb = K / BLOCK, stride = dec_stride(K);
  uint8_t* codes = lds;
  uint8_t* scl = lds + MT * stride;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(xa.v) / sizeof(xa.v[0])); ++i) {
    if (NT * i >= total) break;                        // uniform
    const int q = tid + NT * i;
    float v[8];
    unpack_bf16x8(q < total ? xa.v[i] : make_uint4(0, 0, 0, 0), v);
    int e;
    const uint2 w = quant_quarter(v, e);
    if (q < total) {
      const int r = q / nq, k8 = (q - r * nq) * 8;
      *reinterpret_cast<uint2*>(codes + r * stride + k8) = w;
      if ((k8 & 31) == 0) scl[r * nkb + k8 / BLOCK] = (uint8_t)(e + 127);
    }
  }
}

// The weight operands of a real wave: NPV virtual waves x CPV chunks each.
template <int NPV, int CPV>
struct DecW {
  Operand b[NPV][CPV];
};

// 3. the wave's weight chunks (unconditional: a chunk that does not exist reads the
//    row start and is zeroed)
template <bool PAIRED, int RW, int NPV, int CPV>
__device__ __forceinline__ void dec_w_load(const DecodeArgs& p, int bx, int wave, int lane, DecW<NPV, CPV>& w) {
  const int c16 = lane & 15, kg = lane >> 4;
  const int K = p.K, nkb = K / BLOCK, nch = (K + CHUNK - 1) / CHUNK;
  int mat, n;
  if constexpr (PAIRED) {
    mat = c16 >> 3;
    n = bx * 8 + (c16 & 7);
  } else {
    mat = 0;
    n = bx * 16 + c16;
  }
  // (select, not index: a lane-dependent index into the argument block would be a
  // vector memory load)
  const uint8_t* brow = (mat ? p.w[1] : p.w[0]) + (size_t)n * K;
  const uint8_t* bsc = (mat ? p.ws[1] : p.ws[0]) + (size_t)(n / 32) * nkb;
#pragma unroll
  for (int i = 0; i < NPV; ++i)
#pragma unroll
    for (int cc = 0; cc < CPV; ++cc) {
      const int v = wave + RW * i, c = v + DEC_VW * cc;
      w.b[i][cc] = load_operand(brow, bsc, v < DEC_VW && c < nch ? K : 0, c, kg, true);
    }
}

// 4. the wave's virtual waves: A from LDS (rows >= mt are zero), B from registers;
//    each partial tile to red (after the quantized rows are in LDS)
template <int MT, int RW, int NPV, int CPV>
__device__ __forceinline__ void dec_mfma(const DecodeArgs& p, int mt, int wave, int lane, const DecW<NPV, CPV>& w,
                                         uint8_t* lds) {
  const int c16 = lane & 15, kg = lane >> 4;
  const int K = p.K, nkb = K / BLOCK, nch = (K + CHUNK - 1) / CHUNK, stride = dec_stride(K);
  const uint8_t* codes = lds;
  const uint8_t* scl = lds + MT * stride;
  float* red = reinterpret_cast<float*>(lds + dec_red_offset(MT, K));
#pragma unroll
  for (int i = 0; i < NPV; ++i) {
    const int v = wave + RW * i;
    if (v >= DEC_VW) break;                            // uniform
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int cc = 0; cc < CPV; ++cc) {
      const int c = v + DEC_VW * cc;
      if (c >= nch) break;                             // uniform
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
      const float sa = e8m0_to_f32(A.s), sb = e8m0_to_f32(w.b[i][cc].s);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma_bf16(step_values(A, j, sa), step_values(w.b[i][cc], j, sb), acc);
    }
    if (lane < 16) *reinterpret_cast<float4*>(red + (v * 16 + lane) * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
}

// 3'/4' (a non-PAIRED tile whose 16 weight rows were copied into LDS, wl = rows
//    [16 bx, 16 bx + 16) x K bytes): the E8M0 scales of the wave's chunks (bsc =
//    the tile's scale row, K / 32 bytes), then the partial tiles as dec_mfma forms
//    them -- the same operands, so the same bits.
template <int NPV, int CPV>
__device__ __forceinline__ void dec_wscale(const uint8_t* bsc, int K, int wave, int RW, int lane,
                                           uint32_t (&bs)[NPV][CPV]) {
  const int kg = lane >> 4;
  const int nch = (K + CHUNK - 1) / CHUNK;
#pragma unroll
  for (int i = 0; i < NPV; ++i)
#pragma unroll
    for (int cc = 0; cc < CPV; ++cc) {
      const int v = wave + RW * i, c = v + DEC_VW * cc;
      const bool ok = v < DEC_VW && c < nch && c * CHUNK + BLOCK * kg < K;
      const uint32_t sc = bsc[ok ? 4 * c + kg : 0];
      bs[i][cc] = ok ? sc : E8M0_ONE;
    }
}

template <int MT, int NPV, int CPV>
__device__ __forceinline__ void dec_mfma_wlds(const DecodeArgs& p, int mt, int wave, int RW, int lane,
                                              const uint8_t* wl, const uint32_t (&bs)[NPV][CPV], uint8_t* lds) {
  const int c16 = lane & 15, kg = lane >> 4;
  const int K = p.K, nkb = K / BLOCK, nch = (K + CHUNK - 1) / CHUNK, stride = dec_stride(K);
  const uint8_t* codes = lds;
  const uint8_t* scl = lds + MT * stride;
  float* red = reinterpret_cast<float*>(lds + dec_red_offset(MT, K));
#pragma unroll
  for (int i = 0; i < NPV; ++i) {
    const int v = wave + RW * i;
    if (v >= DEC_VW) break;                            // uniform
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int cc = 0; cc < CPV; ++cc) {
      const int c = v + DEC_VW * cc;
      if (c >= nch) break;                             // uniform
      const int k0 = c * CHUNK + BLOCK * kg;
      // (reads at clamped addresses, then selects: no branch around the LDS reads)
      const bool kin = k0 < K, ain = c16 < mt && kin;
      const int kk = kin ? k0 : 0, ar = ain ? c16 : 0;
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 alo = *reinterpret_cast<const uint4*>(codes + ar * stride + kk);
      const uint4 ahi = *reinterpret_cast<const uint4*>(codes + ar * stride + kk + 16);
      const uint32_t as = scl[ar * nkb + (kin ? 4 * c + kg : 0)];
      const uint4 blo = *reinterpret_cast<const uint4*>(wl + c16 * K + kk);
      const uint4 bhi = *reinterpret_cast<const uint4*>(wl + c16 * K + kk + 16);
      Operand A, B;
      A.lo = ain ? alo : z;
      A.hi = ain ? ahi : z;
      A.s = ain ? as : E8M0_ONE;
      B.lo = kin ? blo : z;
      B.hi = kin ? bhi : z;
      B.s = bs[i][cc];
      const float sa = e8m0_to_f32(A.s), sb = e8m0_to_f32(B.s);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma_bf16(step_values(A, j, sa), step_values(B, j, sb), acc);
    }
    if (lane < 16) *reinterpret_cast<float4*>(red + (v * 16 + lane) * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
}

// 5. column col of token t (< 4): the 16 partial tiles summed in virtual-wave order
__device__ __forceinline__ float dec_total(const uint8_t* lds, int MT, int K, int col, int t) {
  const float* red = reinterpret_cast<const float*>(lds + dec_red_offset(MT, K));
  float s = red[col * 4 + t];
#pragma unroll
  for (int v = 1; v < DEC_VW; ++v) s += red[(v * 16 + col) * 4 + t];
  return s;
}


// ---- the shared expert carried by routed decode launches (one token)
// K (D in gate/up, the shared F in down) runs as the 16 virtual waves above, at most
// two chunks each, so the outputs equal the shared expert's own launches bit for bit.
constexpr int SH_MAX_K = DEC_VW * 2 * CHUNK;   // 4096
constexpr int SH_CPV = 2;

// One shared gate/up tile (8 rows of w1 and of w3) per workgroup of THREADS threads
// (4 or more waves): h [F_sh] bf16 to p.out.  lds: dec_tile_lds(1, K) bytes.
template <int THREADS>
__device__ __forceinline__ void shared_gu_tile(const DecodeArgs& p, int bx, uint8_t* lds) {
  constexpr int RW = THREADS / 64;
  constexpr int NPV = (DEC_VW + RW - 1) / RW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  DecAct<1, THREADS> xa;
  dec_act_load<1, THREADS>(p, 0, 1, tid, xa);
  __builtin_amdgcn_sched_barrier(0);   // the activation loads ahead of the weight loads
  DecW<NPV, SH_CPV> w;
  dec_w_load<true, RW, NPV, SH_CPV>(p, bx, wave, lane, w);
  dec_act_quant<1, THREADS>(p, 1, tid, xa, lds);
  lds_sync();
  dec_mfma<1, RW, NPV, SH_CPV>(p, 1, wave, lane, w, lds);
  lds_sync();
  if (tid < 8) {
    const float g = round_bf16(dec_total(lds, 1, p.K, tid, 0));
    const float u = round_bf16(dec_total(lds, 1, p.K, tid + 8, 0));
    p.out[bx * 8 + tid] = f32_to_bf16(swiglu_h(g, u, p.limit));
  }
}

// The FP8 shared expert of a decode layer (E4M3 weights, E8M0 block-32 scales):
// w1, w3 [F, D] with scales [F / 32, D / 32], w2 [D, F] with [D / 32, F / 32].
struct SharedWeights {
  const uint8_t *w1, *s1, *w3, *s3, *w2, *s2;
  int F;
};

// Standalone one-token decode of the shared expert (shared_fp8.hip): h [F], y [D] bf16.
int launch_decode(const uint16_t* x, const uint8_t* w1, const uint8_t* s1, const uint8_t* w3, const uint8_t* s3,
                  const uint8_t* w2, const uint8_t* s2, int M, int D, int F, float limit, uint16_t* h, uint16_t* y,
                  hipStream_t s);

}  // namespace fp8
}  // namespace cachalot
