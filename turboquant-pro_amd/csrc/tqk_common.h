// Shared device helpers and tables for the gfx950 TurboQuant KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tqk.h"

#define TQK_D 128          // head_dim supported by the GPU path
#define TQK_MAX_G 256      // largest group (flush) size
#define TQK_OBLK 32        // outlier side-list bound granularity (tokens)
#define TQK_NOB 8          // cumulative outlier counts kept per (group slot, head)
// Largest value norm the decode's fp16 PV weights carry: the online softmax
// keeps every weight p <= 4, and p * norm must stay below fp16's 65504.
#define TQK_MAX_VNORM 16376.0f
// Bits of tqk_encode_groups' overflow word
#define TQK_OVF_OUTLIERS 1  // a (group, head) side-list exceeded outlier_cap
#define TQK_OVF_VNORM 2     // a value norm exceeded TQK_MAX_VNORM

// Value codes use the MFMA-tiled byte order when every 16-token tile lies in
// one page and groups are whole 32-token blocks; otherwise per-token rows.
__host__ __device__ __forceinline__ bool v_tiled(int G, int P) {
  return (P % 16 == 0) && (G % 32 == 0);
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

// Key code rows: k_row_bytes(kb) bytes per token.  4-bit keys are the
// reference's byte stream (byte n = rev4(code[2n]) << 4 | rev4(code[2n+1])).
// 3- and 2-bit keys (uniform grid) are four 32-channel chunks of
// k_row_bytes(kb) / 4 bytes; in chunk c the little-endian field i (2*kb bits
// at bit 2*kb*i) is code(32c + 2i) | code(32c + 2i + 1) << kb.  Either way a
// channel pair has one table index: the byte, or the field.
__host__ __device__ __forceinline__ int k_row_bytes(int kb) { return TQK_D * kb / 8; }
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
// to d = 127, each product and sum separately rounded, in d order; u_a[d]
// lives in register d % 8 of lane d / 8 of the 16-lane row.  Plain
// operators, so that the broadcast folds into the multiply as its DPP source
// operand: only for units built with -ffp-contract=off (the encode and the
// block quantizers), where a product and a sum are never fused.
template <int K>
__device__ __forceinline__ void rotate_row_dpp(float& y0, float& y1, const float (&ua)[8],
                                               const float (&ub)[8], const float (&pcol)[TQK_D]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float p0 = dpp_row_bcast<K>(ua[r]) * pcol[8 * K + r];
    const float p1 = dpp_row_bcast<K>(ub[r]) * pcol[8 * K + r];
    y0 = y0 + p0;
    y1 = y1 + p1;
  }
  if constexpr (K + 1 < TQK_D / 8) rotate_row_dpp<K + 1>(y0, y1, ua, ub, pcol);
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
