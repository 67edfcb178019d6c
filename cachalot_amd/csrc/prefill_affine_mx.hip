#include "prefill_mx.h"

namespace cachalot {
namespace {

using namespace decode;
using namespace pmx;

// Affine prefill in groups of 64 (2-bit g64, 3- and 4-bit g64: oQ3e is 3-bit g64) on
// v_mfma_scale_f32_32x32x64_f8f6f4: one instruction per plane covers one 64-element
// half of a K chunk, so a group of 64 is one instruction and nothing is masked (a
// 16 x 16 x 128 instruction holds two such groups).  Reference semantics as
// prefill_mx.hip (expert_affine.py:84-99, the group formula of minimax/codes_qmv.py:86-100).
//
// Built with -mllvm -amdgpu-mfma-vgpr-form=true: the tiles stay in VGPRs, where the
// per-group fold reads them (with AGPR tiles every fold read is a copy).
//
// Operand layout (fp8, measured): lane l holds row (A) or column (B) l & 31; its
// registers 0..3 carry elements 16 (l >> 5) .. + 15 of the 64, registers 4..7 elements 32 + 16 (l >> 5) .. + 15; the scale of block b
// (elements 32 b .. 32 b + 31) of row r comes from lane 32 b + r.  Result register j of
// lane l: row 8 (j / 4) + 4 (l >> 5) + (j & 3), column l & 31.
//
// One 256-thread workgroup = the 64-row M tile x 32 NF weight rows per wave of each of
// NM matrices (gate/up: NM = 2, NF = 1; down: NM = 1, NF = 2); the A ring, the tile
// mapping and the plane writers are those of p3_kernel.
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
constexpr int P4_TB = P3_MT / 32;   // 32-row token blocks

// The tile stays in VGPRs (the fold reads it there); ZERO: the accumulator input is the
// inline constant 0.
template <int OPSEL_A, bool ZERO>
__device__ __forceinline__ f32x16_t mfma32_plane(const i32x8_t& a, const i32x8_t& b, f32x16_t c, uint32_t sa) {
  f32x16_t d;
  if constexpr (ZERO) {
    const f32x16_t z = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, z, 0, 0, OPSEL_A, (int)sa, 0, (int)E8M0_2P9);
  } else {
    d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, OPSEL_A, (int)sa, 0, (int)E8M0_2P9);
  }
  return d;
}

template <int NP>
struct P4Chunk {
  uint4 codes[NP][2];   // per (matrix, weight block) pair and half of the chunk: the lane's two runs
};

// Codes of half h of chunk c for lane half kh: runs at elements 64 h + 16 kh and + 32,
// 2 BITS bytes each, loaded as whole words as in p3_issue_aff.  (The scales and biases
// come in groups of eight, p4_kernel.)
template <int AK, int NM, int NF>
__device__ __forceinline__ void p4_issue(uint8_t* stage, const uint8_t* (&asrc)[P3_ASLOTS], const uint8_t* base,
                                         const int (&woff)[NM], const int (&nrow)[NF], int c, int kh, int wave,
                                         int row_bytes, P4Chunk<NM * NF>& out) {
  constexpr int BITS = ak_bits(AK), CB = 16 * BITS;
  constexpr int LB = BITS == 2 ? 4 : 8;
#pragma unroll
  for (int q = 0; q < P3_ASLOTS; ++q)
    tile::lds_load16_untracked(asrc[q] + (size_t)c * P3_ROWB, stage + (P3_ASLOTS * wave + q) * 1024);
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint8_t* row = base + woff[m] + nrow[f] * row_bytes;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r0 = (2 * BITS * (4 * h + kh)) & ~3, r1 = (2 * BITS * (4 * h + kh) + 4 * BITS) & ~3;
        const int o0 = min(c * CB + r0, row_bytes - LB), o1 = min(c * CB + r1, row_bytes - LB);
        if constexpr (BITS == 2) {
          out.codes[m * NF + f][h] = make_uint4(*reinterpret_cast<const uint32_t*>(row + o0),
                                                *reinterpret_cast<const uint32_t*>(row + o1), 0u, 0u);
        } else {
          const uint2 a = *reinterpret_cast<const uint2*>(row + o0);
          const uint2 b = *reinterpret_cast<const uint2*>(row + o1);
          out.codes[m * NF + f][h] = make_uint4(a.x, a.y, b.x, b.y);
        }
      }
    }
}

// One chunk: per token block and group (half) h, the two plane instructions of every
// pair into a zeroed tile, folded in as acc = fma(s, tile, fma(b, sum x, acc)).  The
// token blocks run one after the other, so one block's tiles are live at a time.
template <int AK, int NP>
__device__ __forceinline__ void p4_compute(const uint8_t* ab, const uint8_t* sbuf, int sbs, const float* sxs,
                                           const P4Chunk<NP>& ch, const uint32_t (&sw)[NP], const uint32_t (&bw)[NP],
                                           int c, int lane, int ntb, int groups, bool f16, f32x16_t (&acc)[NP][P4_TB]) {
  static_assert(ak_group(AK) == 64, "one group per instruction");
  const int r32 = lane & 31, kh = lane >> 5;
  const int nh = min(2, groups - 2 * c);   // the chunk's groups inside the row
  float sc[NP][2], bi[NP][2];
  i32x8_t b[NP][2];   // both halves' operands, built once for the token blocks
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[p][h] = scale_bits_to_f32((uint16_t)(sw[p] >> (16 * h)), f16);
      bi[p][h] = scale_bits_to_f32((uint16_t)(bw[p] >> (16 * h)), f16);
      b[p][h] = aff_code_bytes<ak_bits(AK)>(ch.codes[p][h], kh);
    }
#pragma unroll
  for (int tb = 0; tb < P4_TB; ++tb) {
    if (tb >= ntb) break;
    const int row = tb * 32 + r32;
    const uint8_t* ar = ab + row * P3_ROWB;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h >= nh) break;
      const int c0 = 4 * h + kh, c1 = 4 * h + 2 + kh;   // 16-byte columns of the hi plane
      const uint4 h0 = mx::lds16(ar + ((c0 ^ (row & 15)) << 4));
      const uint4 h1 = mx::lds16(ar + ((c1 ^ (row & 15)) << 4));
      const uint4 l0 = mx::lds16(ar + (((8 + c0) ^ (row & 15)) << 4));
      const uint4 l1 = mx::lds16(ar + (((8 + c1) ^ (row & 15)) << 4));
      const uint32_t sa = *reinterpret_cast<const uint16_t*>(sbuf + row * sbs + (4 * c + 2 * h + kh) * 2);
      const i32x8_t ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
      const i32x8_t alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
      f32x16_t d[NP];
#pragma unroll
      for (int p = 0; p < NP; ++p) d[p] = mfma32_plane<0, true>(ahi, b[p][h], d[p], sa);
#pragma unroll
      for (int p = 0; p < NP; ++p) d[p] = mfma32_plane<1, false>(alo, b[p][h], d[p], sa);
      float sx[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(sxs + (2 * c + h) * P3_MT + tb * 32 + 8 * q + 4 * kh);
        sx[4 * q] = v.x;
        sx[4 * q + 1] = v.y;
        sx[4 * q + 2] = v.z;
        sx[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[p][tb][j] = fmaf(sc[p][h], d[p][j], fmaf(bi[p][h], sx[j], acc[p][tb][j]));
    }
  }
}

template <int AK, int NM, int NF>
__global__ void __launch_bounds__(P3_THREADS) p4_kernel(MxArgs g, int slices) {
  constexpr int GPC = ak_gpc(AK), NP = NM * NF;
  extern __shared__ __align__(16) uint8_t p3_lds[];
  uint8_t* abuf = p3_lds;
  uint8_t* sbuf = p3_lds + P3_STAGES * P3_ABYTES;
  const int sbs = g.sb + 16;
  float* sxs = reinterpret_cast<float*>(sbuf + P3_MT * sbs);   // the tile's group sums [kch * GPC][MT]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31, kh = lane >> 5;
  const int b8 = blockIdx.x >> 3;
  const int slice = b8 % slices;
  const int tile_id = (b8 / slices) * 8 + (int)(blockIdx.x & 7);
  if (tile_id >= g.tiles_n[0]) return;
  const int2 tl = g.tiles[tile_id];
  const int e = tl.x, row0 = tl.y;
  const int rows = min(P3_MT, g.offsets[e + 1] - row0);
  const int ntb = __builtin_amdgcn_readfirstlane((rows + 31) >> 5);
  const int slot = g.slot_table[e];
  constexpr int WN = 32 * NF;                            // weight rows per wave and matrix
  const int nw0 = slice * (P3_WAVES * WN) + WN * wave;
  f32x16_t acc[NP][P4_TB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int tb = 0; tb < P4_TB; ++tb)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[p][tb][j] = 0.0f;
  if (slot >= 0) {
    const int groups = (g.K + ak_group(AK) - 1) / ak_group(AK);
    const int row_bytes = groups * ak_group(AK) * ak_bits(AK) / 8;
    const int sq = g.sb / 16;
    for (int it = threadIdx.x; it < P3_MT * sq; it += P3_THREADS) {
      const int r = it / sq, q = it - r * sq;
      const int rr = row0 + min(r, rows - 1);
      const int src = g.a_gather ? g.a_gather[rr] : rr;
      *reinterpret_cast<uint4*>(sbuf + r * sbs + q * 16) =
          *reinterpret_cast<const uint4*>(g.as + (size_t)src * g.sb + q * 16);
    }
    {
      const int ns = g.kch * GPC;
      for (int it = threadIdx.x; it < P3_MT * ns; it += P3_THREADS) {
        const int ch = it / P3_MT, r = it - ch * P3_MT;
        const int rr = row0 + min(r, rows - 1);
        const int src = g.a_gather ? g.a_gather[rr] : rr;
        sxs[it] = g.asum[(size_t)src * ns + ch];
      }
    }
    const uint8_t* asrc[P3_ASLOTS];
#pragma unroll
    for (int q = 0; q < P3_ASLOTS; ++q) {
      const int S = 64 * (P3_ASLOTS * wave + q) + lane;
      const int r = S >> 4;
      const int col = (S & 15) ^ (r & 15);
      const int rr = row0 + min(r, rows - 1);
      const int src = g.a_gather ? g.a_gather[rr] : rr;
      asrc[q] = g.ap + (size_t)src * g.kch * P3_ROWB + col * 16;
    }
    const uint8_t* base = g.pool + (int64_t)slot * g.L.record_bytes;
    const int tq[2] = {NM == 2 ? 0 : 3, 6};   // w1, w3 (gate/up) or w2 (down)
    int woff[NM], soff[NM], boff[NM], nrow[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) nrow[f] = min(nw0 + 32 * f + r32, g.N - 1);   // rows past N: clamped (discarded)
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      woff[m] = (int)g.L.off[tq[m]];
      soff[m] = (int)g.L.off[tq[m] + 1];
      boff[m] = (int)g.L.off[tq[m] + 2];
    }
    const int nch = g.kch;
    // Scales and biases, eight groups (four chunks) per 16-byte load: lanes kh = 0 the
    // scale row, kh = 1 the bias row, exchanged across the wave's halves per chunk.  One
    // line of each row then serves 16 chunks from 4 loads (a load per chunk and row kept
    // the rows' lines resident for the whole K loop, more than L2 holds).  A last group
    // of eight past the row reads what follows it in the record (the host checks that
    // something does); those groups are never used.
    const int nq = (groups + 7) / 8;
    uint4 sg[2][NP];
    auto load_sg = [&](int q, uint4(&dst)[NP]) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          dst[m * NF + f] =
              *reinterpret_cast<const uint4*>(base + (kh ? boff[m] : soff[m]) + (nrow[f] * groups + 8 * q) * 2);
    };
    load_sg(0, sg[0]);
    P4Chunk<NP> ring[P3_STAGES];
    p4_issue<AK, NM, NF>(abuf, asrc, base, woff, nrow, 0, kh, wave, row_bytes, ring[0]);
    for (int c0 = 0; c0 < nch; c0 += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u;
        // this wave's loads of chunk c have landed (the last code load is consumed here;
        // the scale group, issued before it, first), then every wave's; the first barrier
        // also publishes the staged sums
        asm volatile("" ::"v"(ring[u % 2].codes[NP - 1][1].w) : "memory");
        lds_sync();
        if ((u + 1) % 4 == 0) load_sg(min((c + 1) / 4, nq - 1), sg[((u + 1) / 4) % 2]);
        p4_issue<AK, NM, NF>(abuf + ((u + 1) % 2) * P3_ABYTES, asrc, base, woff, nrow, min(c + 1, nch - 1), kh, wave,
                             row_bytes, ring[(u + 1) % 2]);
        if (c < nch) {
          uint32_t sw[NP], bw[NP];
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const uint4& v = sg[(u / 4) % 2][p];
            const uint32_t mine = (u % 4) == 0 ? v.x : (u % 4) == 1 ? v.y : (u % 4) == 2 ? v.z : v.w;
            const uint32_t other = (uint32_t)__shfl_xor((int)mine, 32, 64);
            sw[p] = kh ? other : mine;
            bw[p] = kh ? mine : other;
          }
          p4_compute<AK, NP>(abuf + (u % 2) * P3_ABYTES, sbuf, sbs, sxs, ring[u % 2], sw, bw, c, lane, ntb, groups,
                             g.L.f16, acc);
        }
      }
    }
    tile::wait_vmem();
  }
  if constexpr (NM == 2) {
    float* red = reinterpret_cast<float*>(abuf);   // [P3_WAVES][P3_MT]
    lds_sync();
    const int n = nw0 + r32;
#pragma unroll
    for (int tb = 0; tb < P4_TB; ++tb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int tr = tb * 32 + 8 * (j / 4) + 4 * kh + (j & 3);   // the same in the 32 lanes of a half
        if (tr >= rows) continue;
        const int prow = row0 + tr;
        const float wr = g.row_w[prow];
        float gv = round_bf16(acc[0][tb][j]);
        float uv = round_bf16(acc[1][tb][j]);
        if (g.limit > 0.0f) {
          uv = fminf(fmaxf(uv, -g.limit), g.limit);
          gv = fminf(gv, g.limit);
        }
        const float hv = n < g.N ? round_bf16((silu_f32(gv) * uv) * wr) : 0.0f;
        float m = mx::row16_max(fabsf(hv));
        m = fmaxf(m, xor_f<16>(m));
        const int E = plane_exp(m);
        const float s = hv * __uint_as_float((uint32_t)(127 - E) << 23);
        const uint32_t hi = mx::f32_to_e4m3(s);
        const uint32_t lo = mx::f32_to_e4m3((s - mx::e4m3_to_f32(hi)) * 16.0f);
        uint8_t* p = g.hp + ((size_t)prow * g.hkch + (n >> 7)) * P3_ROWB + (n & 127);
        p[0] = (uint8_t)hi;
        p[128] = (uint8_t)lo;
        float hs = row16_sum(hv);
        hs = hs + xor_f<16>(hs);
        if (r32 == 0) {
          const uint32_t sc = (uint32_t)(E + 127) | ((uint32_t)(E + 123) << 8);
          *reinterpret_cast<uint16_t*>(g.hs + (size_t)prow * g.hsb + (nw0 / 32) * 2) = (uint16_t)sc;
          red[wave * P3_MT + tr] = hs;
        }
      }
    lds_sync();
    if ((int)threadIdx.x < rows) {
      const int tr = threadIdx.x;
#pragma unroll
      for (int h = 0; h < GPC; ++h) {
        float t = 0.0f;
#pragma unroll
        for (int w = h * P3_WAVES / GPC; w < (h + 1) * P3_WAVES / GPC; ++w) t = t + red[w * P3_MT + tr];
        g.hsum[(size_t)(row0 + tr) * g.hkch * GPC + slice * GPC + h] = t;
      }
    }
  } else {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int n = nw0 + 32 * f + r32;
      if (n >= g.N) continue;
#pragma unroll
      for (int tb = 0; tb < P4_TB; ++tb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int tr = tb * 32 + 8 * (j / 4) + 4 * kh + (j & 3);
          if (tr >= rows) continue;
          const int rr = row0 + tr;
          g.y[((size_t)g.row_token[rr] * g.k + g.row_slot[rr]) * g.N + n] = f32_to_bf16(acc[f][tb][j]);
        }
    }
  }
}

template <int AK>
int launch_pair(const MxArgs& gu, int s_gu, size_t lds_gu, const MxArgs& dn, int s_dn, size_t lds_dn, int tiles8,
                hipStream_t s) {
  auto kgu = p4_kernel<AK, 2, 1>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kgu), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_gu) != hipSuccess)
    return fail(CACHALOT_EHIP, "prefill (block-scaled): cannot grant %zu bytes of LDS", lds_gu);
  hipLaunchKernelGGL(kgu, dim3(s_gu * tiles8), dim3(P3_THREADS), lds_gu, s, gu, s_gu);
  int rc = check_launch("p4_kernel<2,1>");
  if (rc) return rc;
  auto kdn = p4_kernel<AK, 1, 2>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kdn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds_dn) != hipSuccess)
    return fail(CACHALOT_EHIP, "prefill (block-scaled): cannot grant %zu bytes of LDS", lds_dn);
  hipLaunchKernelGGL(kdn, dim3(s_dn * tiles8), dim3(P3_THREADS), lds_dn, s, dn, s_dn);
  return check_launch("p4_kernel<1,2>");
}

}  // namespace

// The gate/up and down launches over the x planes and sums prefill_mx.hip has written
// (grids as p3_kernel's: s slices x the tile list rounded up to 8).
int launch_prefill_affine_g64(int ak, const pmx::MxArgs& gu, int s_gu, size_t lds_gu, const pmx::MxArgs& dn,
                              int s_dn, size_t lds_dn, int tiles8, hipStream_t s) {
  if (ak == ak_aff(2, 64)) return launch_pair<ak_aff(2, 64)>(gu, s_gu, lds_gu, dn, s_dn, lds_dn, tiles8, s);
  if (ak == ak_aff(3, 64)) return launch_pair<ak_aff(3, 64)>(gu, s_gu, lds_gu, dn, s_dn, lds_dn, tiles8, s);
  if (ak == ak_aff(4, 64)) return launch_pair<ak_aff(4, 64)>(gu, s_gu, lds_gu, dn, s_dn, lds_dn, tiles8, s);
  return fail(CACHALOT_EINVAL, "prefill (block-scaled): weight kind %d has no 64-element groups", ak);
}

}  // namespace cachalot
