// Shared device helpers and tables for the gfx950 TurboQuant KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tqk.h"

#define TQK_D 128          // head_dim of the MFMA decode (other head dims run the VALU decode)
#define TQK_MAX_G 256      // largest group (flush) size
#define TQK_OBLK 32        // outlier side-list bound granularity (tokens)
#define TQK_NOB 8          // cumulative outlier counts kept per (group slot, head)
// Largest value norm the decode's fp16 PV weights carry: the online softmax
// keeps every weight p <= 4, and p * norm must stay below fp16's 65504.
#define TQK_MAX_VNORM 16376.0f
// Bits of tqk_encode_groups' overflow word
#define TQK_OVF_OUTLIERS 1  // a (group, head) side-list exceeded outlier_cap
#define TQK_OVF_VNORM 2     // a value norm exceeded TQK_MAX_VNORM

// head dims the kernels are built for
__host__ __device__ __forceinline__ bool head_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }

// Value codes use the MFMA-tiled byte order when the MFMA decode serves the
// cache (head_dim 128, fp16 inputs), every 16-token tile lies in one page and
// groups are whole 32-token blocks; otherwise per-token rows.
__host__ __device__ __forceinline__ bool v_tiled(int G, int P, int D, int f32) {
  return D == TQK_D && !f32 && (P % 16 == 0) && (G % 32 == 0);
}

// Byte offset of the value-code unit holding tokens [4*lg, 4*lg+4) of a
// 16-token tile and channels [8*c, 8*c+8), relative to the tile start.
// A unit is vrow/4 bytes (12 for 3-bit, 16 for 4-bit codes).
__host__ __device__ __forceinline__ int v_unit_offset(int lg, int c, int vrow) {
  return (16 * lg + c) * (vrow / 4);
}
// Bit position, inside a unit, of the code of token u (0..3 within the unit)
// and channel nt (0..7 within the unit): codes of the token pairs (0,1) and
// (2,3) of one channel sit next to each other as one 2*vb-bit field.
__host__ __device__ __forceinline__ int v_unit_bit(int u, int nt, int vb) {
  return (2 * nt + (u >> 1)) * (2 * vb) + (u & 1) * vb;
}

// NormalFloat-4 levels, turboquant_pro/per_channel_kv.py:64-84.
// Key level of code c: NF4 for key_grid 0, the code itself for uniform keys
__device__ __forceinline__ float key_level(int grid, uint32_t c);
__constant__ static const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};
__device__ __forceinline__ float key_level(int grid, uint32_t c) {
  return grid ? (float)c : kNF4[c];
}

__device__ __forceinline__ float h2f(uint16_t x) {
  return (float)__builtin_bit_cast(_Float16, x);
}
__device__ __forceinline__ uint16_t f2h(float x) {  // round to nearest even
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// 4-bit nibble bit reversal: the key stream stores each code LSB-first inside
// MSB-first bytes (turboquant_pro/per_channel_kv.py:87-93), so byte n holds
// rev4(code[2n]) << 4 | rev4(code[2n+1]).
__host__ __device__ __forceinline__ uint32_t rev4(uint32_t x) {
  return ((x & 1u) << 3) | ((x & 2u) << 1) | ((x & 4u) >> 1) | ((x & 8u) >> 3);
}

// Key code rows: k_row_bytes(kb, D) bytes per token.  4-bit keys are the
// reference's byte stream (byte n = rev4(code[2n]) << 4 | rev4(code[2n+1])).
// 3- and 2-bit keys (uniform grid) are D / 32 chunks of 32 channels, 4 * kb
// bytes each; in chunk c the little-endian field i (2*kb bits at bit 2*kb*i)
// is code(32c + 2i) | code(32c + 2i + 1) << kb.  Either way a channel pair has
// one table index: the byte, or the field.
__host__ __device__ __forceinline__ int k_row_bytes(int kb, int D) { return D * kb / 8; }
// table index of channel pair `pair` (channels 2*pair, 2*pair + 1) of a row
// given as little-endian dwords
__device__ __forceinline__ uint32_t k_pair_index(const uint32_t* rw, int kb, int pair) {
  if (kb == 4) return (rw[pair >> 2] >> (8 * (pair & 3))) & 0xFFu;
  const int o = (pair >> 4) * (32 * kb) + 2 * kb * (pair & 15);  // bit offset in the row (32 channels a chunk)
  const int w = o >> 5, sh = o & 31;
  uint32_t v = rw[w] >> sh;
  if (sh + 2 * kb > 32) v |= rw[w + 1] << (32 - sh);
  return v & ((1u << (2 * kb)) - 1u);
}
// the two codes of a table index
__host__ __device__ __forceinline__ uint32_t k_code_even(uint32_t f, int kb) {
  return kb == 4 ? rev4(f >> 4) : (f & ((1u << kb) - 1u));
}
__host__ __device__ __forceinline__ uint32_t k_code_odd(uint32_t f, int kb) {
  return kb == 4 ? rev4(f & 15u) : (f >> kb);
}

// Number of flushed groups after `len` appends: the first flush fires at
// hot_window + 1 tokens, then every G tokens (turboquant_pro/core.py:1006-1016).
__host__ __device__ __forceinline__ int n_groups_of(int len, int hot_window, int G) {
  return (len <= hot_window) ? 0 : (len - (hot_window + 1)) / G + 1;
}

// Row index of token t (absolute position in its sequence) for kv head h in
// the page pool.
__device__ __forceinline__ size_t page_row(const int32_t* __restrict__ block_table, int max_pages,
                                           int b, int t, int P, int n_pages, int h) {
  // head-major pages: row of token t of sequence b in head h's region
  const int phys = block_table[(size_t)b * max_pages + t / P];
  return ((size_t)h * n_pages + phys) * P + (t % P);
}

// Lane I of each 16-lane row, broadcast to the row (DPP row_newbcast).
template <int I>
__device__ __forceinline__ float dpp_row_bcast(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x150 + I, 0xF, 0xF, true));
}

// y0 += u_a[d] * pcol[d], y1 += u_b[d] * pcol[d] for d = 8K .. 8K + 7 and on
// to d = 8 NL - 1, each product and sum separately rounded, in d order; u_a[d]
// lives in register d % 8 of lane d / 8 of the 16-lane row (NL <= 16 lanes
// hold a chunk of 8 NL channels).  Plain operators, so that the broadcast
// folds into the multiply as its DPP source operand: only for units built
// with -ffp-contract=off (the encode and the block quantizers), where a
// product and a sum are never fused.
template <int K, int NL, int N>
__device__ __forceinline__ void rotate_row_dpp(float& y0, float& y1, const float (&ua)[8],
                                               const float (&ub)[8], const float (&pcol)[N]) {
  static_assert(NL <= 16 && 8 * NL <= N, "a chunk spans at most one 16-lane row");
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float p0 = dpp_row_bcast<K>(ua[r]) * pcol[8 * K + r];
    const float p1 = dpp_row_bcast<K>(ub[r]) * pcol[8 * K + r];
    y0 = y0 + p0;
    y1 = y1 + p1;
  }
  if constexpr (K + 1 < NL) rotate_row_dpp<K + 1, NL>(y0, y1, ua, ub, pcol);
}

// PolarQuant codes of nb <= 64 normalised rows u_s[0..nb) for the rotated
// channel ecol this lane owns: y_e = sum_d u_d * pi[e][d] (sequential in d,
// separately rounded, as the reference's einsum), code = #{ boundaries < y_e }
// (a NaN y_e takes the last code, as searchsorted does), written to
// vc[j][ecol].  Lane layout: the lane's 16-lane row (rt = lane >> 4) takes
// tokens j0 + rt and j0 + 4 + rt of each 8-token step; lane li = lane & 15
// holds eight channels of the row and broadcasts them to its row by DPP.
// Rows longer than 128 channels go in 128-channel chunks, the column chunk in
// registers and every step's sums carried from chunk to chunk.  The 64 lanes
// of the wave must all run it (the broadcasts read other lanes).
template <int D, int VB>
__device__ __forceinline__ void rotate_codes(const float* __restrict__ pi, const float (*u_s)[D],
                                             int nb, int ecol, int lane, const float (&bnd)[15],
                                             uint8_t (*vc)[D]) {
  constexpr int CH = D < 128 ? D : 128;  // channels per chunk
  const int rt = lane >> 4, lc = (lane & 15) % (CH / 8);
  auto load_u = [&](int ja, int jb, int c, float (&ua)[8], float (&ub)[8]) {
    const float4* ra = reinterpret_cast<const float4*>(&u_s[min(ja, nb - 1)][CH * c + 8 * lc]);
    const float4* rb = reinterpret_cast<const float4*>(&u_s[min(jb, nb - 1)][CH * c + 8 * lc]);
    const float4 a0 = ra[0], a1 = ra[1], b0 = rb[0], b1 = rb[1];
    ua[0] = a0.x; ua[1] = a0.y; ua[2] = a0.z; ua[3] = a0.w;
    ua[4] = a1.x; ua[5] = a1.y; ua[6] = a1.z; ua[7] = a1.w;
    ub[0] = b0.x; ub[1] = b0.y; ub[2] = b0.z; ub[3] = b0.w;
    ub[4] = b1.x; ub[5] = b1.y; ub[6] = b1.z; ub[7] = b1.w;
  };
  auto store = [&](int ja, int jb, float y0, float y1) {
    uint32_t c0 = 0, c1 = 0;
#pragma unroll
    for (int k = 0; k < (1 << VB) - 1; ++k) {
      c0 += (bnd[k] < y0) ? 1u : 0u;
      c1 += (bnd[k] < y1) ? 1u : 0u;
    }
    if (y0 != y0) c0 = (1u << VB) - 1u;
    if (y1 != y1) c1 = (1u << VB) - 1u;
    if (ja < nb) vc[ja][ecol] = (uint8_t)c0;
    if (jb < nb) vc[jb][ecol] = (uint8_t)c1;
  };
  auto load_col = [&](int c, float (&pcol)[CH]) {
#pragma unroll
    for (int k = 0; k < CH / 4; ++k) {
      const float4 p4 = reinterpret_cast<const float4*>(pi + (size_t)ecol * D + CH * c)[k];
      pcol[4 * k] = p4.x;
      pcol[4 * k + 1] = p4.y;
      pcol[4 * k + 2] = p4.z;
      pcol[4 * k + 3] = p4.w;
    }
  };
  if constexpr (D <= 128) {
    float pcol[CH];
    load_col(0, pcol);
    for (int j0 = 0; j0 < nb; j0 += 8) {
      const int ja = j0 + rt, jb = j0 + 4 + rt;
      float ua[8], ub[8];
      load_u(ja, jb, 0, ua, ub);
      float y0 = 0.f, y1 = 0.f;
      rotate_row_dpp<0, CH / 8>(y0, y1, ua, ub, pcol);
      // keeps the sums out of the conditional stores: sunk into them, the
      // multiplies would leave their broadcasts behind as separate moves
      asm volatile("" : "+v"(y0), "+v"(y1));
      store(ja, jb, y0, y1);
    }
  } else {
    float ya[8], yb[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) ya[st] = yb[st] = 0.f;
    for (int c = 0; c < D / CH; ++c) {
      float pcol[CH];
      load_col(c, pcol);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (8 * st < nb) {
          float ua[8], ub[8];
          load_u(8 * st + rt, 8 * st + 4 + rt, c, ua, ub);
          rotate_row_dpp<0, CH / 8>(ya[st], yb[st], ua, ub, pcol);
          asm volatile("" : "+v"(ya[st]), "+v"(yb[st]));
        }
      }
    }
#pragma unroll
    for (int st = 0; st < 8; ++st) store(8 * st + rt, 8 * st + 4 + rt, ya[st], yb[st]);
  }
}

// Sum of squares of a D-channel row in NumPy's pairwise order (the L2 norm of
// np.linalg.norm over a contiguous row), four threads per row: thread q
// (= lane & 3, the four consecutive lanes of the row) holds x0[m], x1[m] =
// channels 8m + 2q, 8m + 2q + 1.  NumPy sums a run of n <= 128 values with
// eight strided accumulators r[k] (channels = k mod 8, in order) combined as
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)); a longer run is split into
// halves (at a multiple of 8) summed apart and added, so D = 256 is the two
// 128-channel halves.  Every product and sum is separately rounded.
template <int D>
__device__ __forceinline__ float pairwise_sumsq(const float (&x0)[D / 8], const float (&x1)[D / 8],
                                                int q) {
  constexpr int M = D > 128 ? 16 : D / 8;  // 8-channel steps per pairwise block
  float ss = 0.f;
#pragma unroll
  for (int blk = 0; blk < D / 8 / M; ++blk) {
    float r0 = __fmul_rn(x0[M * blk], x0[M * blk]), r1 = __fmul_rn(x1[M * blk], x1[M * blk]);
#pragma unroll
    for (int m = 1; m < M; ++m) {
      r0 = __fadd_rn(r0, __fmul_rn(x0[M * blk + m], x0[M * blk + m]));
      r1 = __fadd_rn(r1, __fmul_rn(x1[M * blk + m], x1[M * blk + m]));
    }
    // pairwise tree ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7))
    const float pa = __fadd_rn(r0, r1);
    const float po = __shfl_xor(pa, 1, 4);
    const float pb = (q & 1) ? __fadd_rn(po, pa) : __fadd_rn(pa, po);
    const float pbo = __shfl_xor(pb, 2, 4);
    const float bs = (q & 2) ? __fadd_rn(pbo, pb) : __fadd_rn(pb, pbo);
    ss = blk == 0 ? bs : __fadd_rn(ss, bs);
  }
  return ss;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
