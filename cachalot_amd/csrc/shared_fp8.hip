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
#include "fp8_common.h"

namespace cachalot {
namespace fp8 {

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
// Few tokens (M <= DEC_MT per workgroup tile), two launches of the decode tile
// (fp8_common.h), 16 waves each, one virtual wave per wave:
//   gate/up (PAIRED): 8 rows of w1 and the same 8 rows of w3; the epilogue forms
//     h = bf16(silu(min(g, L)) * clip(u, -L, L)) from the bf16-rounded g and u of
//     each row and writes h [M, F] bf16;
//   down: 16 rows of w2 over act_quant(h), y [M, D] bf16.
// The activation loads are issued first and the weight loads right after, so
// waiting for the activations leaves the weight stream in flight while the
// rows are quantized.
constexpr int DEC_CPV = 3;   // chunks per virtual wave: K <= 16 * 3 * 128 = DEC_MAX_K (and beyond)
static_assert(DEC_VW * DEC_CPV * CHUNK >= DEC_MAX_K, "chunks per virtual wave");

template <bool PAIRED, int CPV>
__global__ __launch_bounds__(DEC_VW * 64) void decode_kernel(DecodeArgs p) {
  constexpr int NT = DEC_VW * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.y * DEC_MT, mt = min(DEC_MT, p.M - t0);
  DecAct<DEC_MT, NT> xa;
  dec_act_load<DEC_MT, NT>(p, t0, mt, tid, xa);
  __builtin_amdgcn_sched_barrier(0);   // keep the activation loads ahead of the weight loads
  DecW<1, CPV> w;
  dec_w_load<PAIRED, DEC_VW, 1, CPV>(p, blockIdx.x, wave, lane, w);
  dec_act_quant<DEC_MT, NT>(p, mt, tid, xa, lds);
  lds_sync();
  dec_mfma<DEC_MT, DEC_VW, 1, CPV>(p, mt, wave, lane, w, lds);
  __syncthreads();
  const int j = tid & 15, i = tid >> 4;
  if (i >= mt) return;
  if constexpr (PAIRED) {
    if (j >= 8) return;
    const float g = round_bf16(dec_total(lds, DEC_MT, p.K, j, i)), u = round_bf16(dec_total(lds, DEC_MT, p.K, j + 8, i));
    p.out[(size_t)(t0 + i) * p.ldo + blockIdx.x * 8 + j] = f32_to_bf16(swiglu_h(g, u, p.limit));
  } else {
    p.out[(size_t)(t0 + i) * p.ldo + blockIdx.x * 16 + j] = f32_to_bf16(dec_total(lds, DEC_MT, p.K, j, i));
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

// ------------------------------------------------------------ many-token GEMM ---
// One 512-thread workgroup = a 128-token x 256-row tile of one matrix; wave (wm, wn),
// wm < 2, wn < 4, owns tokens [64 wm, +64) x rows [64 wn, +64) as 4 x 4 tiles of
// 16 x 16.  K runs in stages of one 32-element block (one E8M0 scale per row and
// stage).  The tiles stay E4M3 bytes in LDS (rows 40 bytes apart, so the 16 rows of a
// fragment fall on distinct banks) with their scale bytes beside them; a wave converts
// each fragment as it reads it (8 values per lane, scale folded in: exact) for
// v_mfma_f32_16x16x32_bf16.  Two LDS buffers, GM_RING blocks of bytes in registers
// (the loads run that many blocks ahead); 123 VGPRs, four waves per SIMD.  Rows past
// M and N read row 0 (masked at the store).
// Measured at M = 4096 (the whole expert, ~450 us against 620 us for 64 x 64 tiles
// read straight from global memory): bf16 tiles in LDS, 64 x 128 wave tiles, two
// waves per SIMD and one to three blocks of prefetch all landed within 450-467 us,
// with the matrix cores ~28 % busy.
constexpr int GM_TM = 128;                      // tokens per tile
constexpr int GM_TN = 256;                      // weight rows per tile
constexpr int GM_ROWB = BLOCK + 8;              // bytes per LDS row: 32 E4M3 + padding
constexpr int GM_STAGE = (GM_TM + GM_TN) * GM_ROWB + GM_TM + GM_TN;   // rows, then one scale byte per row

constexpr int GM_THREADS = 512;
#ifndef CACHALOT_GM_RING
#define CACHALOT_GM_RING 2
#endif
constexpr int GM_RING = CACHALOT_GM_RING;       // blocks of bytes in registers
__global__ __launch_bounds__(GM_THREADS) __attribute__((amdgpu_waves_per_eu(4))) void gemm_kernel(LinearArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t glds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int nt = (p.N + GM_TN - 1) / GM_TN;
  const int mat = blockIdx.x / nt, n0 = (blockIdx.x - mat * nt) * GM_TN;
  const int t0 = blockIdx.y * GM_TM;
  const int K = p.K, nkb = K / BLOCK;
  const uint8_t* w = mat ? p.w[1] : p.w[0];
  const uint8_t* ws = mat ? p.ws[1] : p.ws[0];

  // staged by this thread: 8 bytes of A row (tid / 4) at byte 8 (tid % 4) of the
  // block, and 16 bytes of B row (tid / 2) at byte 16 (tid % 2)
  const int ar = tid >> 2, ah = tid & 3, br = tid >> 1, bh = tid & 1;
  const int at = t0 + ar, bn = n0 + br;
  const uint8_t* arow = p.a + (size_t)(at < p.M ? at : 0) * K + 8 * ah;
  const uint8_t* asc = p.ae + (size_t)(at < p.M ? at : 0) * nkb;
  const uint8_t* brow = w + (size_t)(bn < p.N ? bn : 0) * K + 16 * bh;
  const uint8_t* bsc = ws + (size_t)((bn < p.N ? bn : 0) / 32) * nkb;
  struct Raw {
    uint2 a;
    uint4 b;
    uint32_t sa, sb;
  };
  // blocks past K re-read the last one (unconditional loads; never stored)
  auto load = [&](int kb, Raw& r) {
    const int k = BLOCK * min(kb, nkb - 1);
    r.a = *reinterpret_cast<const uint2*>(arow + k);
    r.b = *reinterpret_cast<const uint4*>(brow + k);
    r.sa = asc[k / BLOCK];
    r.sb = bsc[k / BLOCK];
  };
  auto store = [&](const Raw& r, uint8_t* buf) {
    *reinterpret_cast<uint2*>(buf + ar * GM_ROWB + 8 * ah) = r.a;
    uint2* db = reinterpret_cast<uint2*>(buf + (GM_TM + br) * GM_ROWB + 16 * bh);
    db[0] = make_uint2(r.b.x, r.b.y);
    db[1] = make_uint2(r.b.z, r.b.w);
    uint8_t* sc = buf + (GM_TM + GM_TN) * GM_ROWB;
    if (ah == 0) sc[ar] = (uint8_t)r.sa;
    if (bh == 0) sc[GM_TM + br] = (uint8_t)r.sb;
  };
  // the 8 values of lane (fr, fg) of a fragment whose 16 rows start at LDS row `row0`
  auto frag = [&](const uint8_t* buf, int row, int fg) {
    const uint2 v = *reinterpret_cast<const uint2*>(buf + row * GM_ROWB + 8 * fg);
    const uint32_t sc = buf[(GM_TM + GM_TN) * GM_ROWB + row];
    return to_bf16x8(v.x, v.y, e8m0_to_f32(sc));
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int fr = lane & 15, fg = lane >> 4;   // fragment row / column and k group
  // a ring of GM_RING blocks in registers, two in LDS; GM_RING blocks per trip so the
  // ring index is a constant
  Raw ring[GM_RING];
#pragma unroll
  for (int r = 0; r < GM_RING; ++r) load(r, ring[r]);
  store(ring[0], glds);
  __syncthreads();
  for (int kb0 = 0; kb0 < nkb; kb0 += GM_RING) {
#pragma unroll
    for (int u = 0; u < GM_RING; ++u) {
      const int kb = kb0 + u;
      if (kb < nkb) {
        const uint8_t* buf = glds + (kb & 1) * GM_STAGE;
        load(kb + GM_RING, ring[u]);   // the slot of block kb, already in LDS
        bf16x8_t af[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = frag(buf, 64 * wm + 16 * i + fr, fg);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8_t bfr = frag(buf, GM_TM + 64 * wn + 16 * j + fr, fg);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16(af[i], bfr, acc[i][j]);
        }
        if (kb + 1 < nkb) store(ring[(u + 1) % GM_RING], glds + ((kb + 1) & 1) * GM_STAGE);
        __syncthreads();
      }
    }
  }
  // D[r][c] of a 16 x 16 tile: lane c + 16 (r / 4), register r % 4
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + 64 * wn + 16 * j + fr;
    if (n >= p.N) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = t0 + 64 * wm + 16 * i + 4 * fg + v;
        if (t < p.M) p.out[(size_t)t * p.ldo + mat * p.N + n] = f32_to_bf16(acc[i][j][v]);
      }
  }
}

// Tile choice: token-tiled GEMV (one 16-token tile per workgroup, 8 chunks of
// every wave in flight) for decode-sized M; 128 x 128 LDS tiles for many tokens.
int launch_linear(const LinearArgs& a, int nmat, hipStream_t s) {
  if (a.M > 64) {
    const dim3 grid((unsigned)(nmat * ((a.N + GM_TN - 1) / GM_TN)), (unsigned)((a.M + GM_TM - 1) / GM_TM));
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            2 * GM_STAGE) != hipSuccess)
      return fail(CACHALOT_EHIP, "fp8 linear: cannot grant %d bytes of LDS", 2 * GM_STAGE);
    hipLaunchKernelGGL(gemm_kernel, grid, dim3(GM_THREADS), 2 * GM_STAGE, s, a);
  } else {
    const dim3 grid((unsigned)(nmat * a.N / 16), (unsigned)((a.M + 15) / 16));
    hipLaunchKernelGGL((linear_kernel<1, 1, 8>), grid, dim3(256), 0, s, a);
  }
  return check_launch("fp8 linear");
}

// Decode (M <= DEC_MT): gate/up + SwiGLU -> h [M, F] bf16 (in the gu region), down -> y.
template <int CPV>
int launch_decode_cpv(const DecodeArgs& gu, const DecodeArgs& dn, hipStream_t s) {
  const dim3 grid_gu((unsigned)(gu.N / 8), (unsigned)((gu.M + DEC_MT - 1) / DEC_MT));
  hipLaunchKernelGGL((decode_kernel<true, CPV>), grid_gu, dim3(64 * DEC_VW), dec_tile_lds(DEC_MT, gu.K), s, gu);
  if (int rc = check_launch("fp8 decode gate/up")) return rc;
  const dim3 grid_dn((unsigned)(dn.N / 16), (unsigned)((dn.M + DEC_MT - 1) / DEC_MT));
  hipLaunchKernelGGL((decode_kernel<false, CPV>), grid_dn, dim3(64 * DEC_VW), dec_tile_lds(DEC_MT, dn.K), s, dn);
  return check_launch("fp8 decode down");
}

int launch_decode(const uint16_t* x, const uint8_t* w1, const uint8_t* s1, const uint8_t* w3, const uint8_t* s3,
                  const uint8_t* w2, const uint8_t* s2, int M, int D, int F, float limit, uint16_t* h, uint16_t* y,
                  hipStream_t s) {
  const DecodeArgs gu{x, D, {w1, w3}, {s1, s3}, M, F, D, limit, h, F};
  const DecodeArgs dn{h, F, {w2, w2}, {s2, s2}, M, D, F, limit, y, D};
  const int nch = (std::max(D, F) + CHUNK - 1) / CHUNK;   // chunks of the longer K
  if (nch <= DEC_VW) return launch_decode_cpv<1>(gu, dn, s);
  if (nch <= 2 * DEC_VW) return launch_decode_cpv<2>(gu, dn, s);
  return launch_decode_cpv<3>(gu, dn, s);
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
