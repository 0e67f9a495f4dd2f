// Fused decode-step attention over the two-tier TurboQuant KV cache (gfx950).
//
// One workgroup per (split, kv head, sequence).  A split covers a run of coded
// groups or a slice of the fp16 hot window and produces an unnormalised
// online-softmax state (m, l, acc) for each of the GQ query heads that share
// the kv head (turboquant_pro/kv_kernel.py:255-316 is the reference's M4
// per-(head, split) form; here every query head of a GQA group reuses one
// pass over the codes).  Coded groups are attended in code space:
//   score_t = (sum_j (q_j * a_j) * NF4[code_tj] + sum_j q_j * mu_j
//              + sum_{outliers (t,j)} q_j * (val - dense_tj)) * sm_scale
//   acc     = sum_t p_t * ||v_t|| * cent[vcode_t]            (rotated space)
// (turboquant_pro/kv_fused_pck.py:196-236).  tqk_merge then combines the
// splits, rotates the coded part back with one D x D product per query head
// and adds the hot-window part (turboquant_pro/kv_fused.py:139-153).
#include <atomic>
#include <mutex>

#include "tqk_common.h"

namespace {

struct DecodeArgs {
  tqk_cache_desc d;
  tqk_cache_ptrs p;
  const void* q;  // fp16, or fp32 (input_f32: VALU kernel only)
  const int32_t* seq_lens;
  float* pm;    // [batch][Hq][n_splits]
  float* pl;    // [batch][Hq][n_splits]
  float* pacc;  // [batch][Hq][n_splits][D]
  int n_cold_splits;
  int n_hot_splits;
  int groups_per_split;
  // MFMA kernel, splits of fewer groups than waves: each wave takes this many
  // consecutive blocks of the split (0: each wave takes whole groups, every
  // eighth group of the split)
  int wave_blocks;
  int hot_per_split;
  int split_base;  // added to blockIdx.x (hot-only launches start after the coded splits)
  int batch;
  // MFMA kernel: 1 when the grid takes more than one round of CUs, so that
  // the order in which (seq, split) items start matters (longest first)
  int reorder;
  // in-kernel merge (MFMA kernel): the output, or nullptr to leave the
  // partials to tqk_merge, and one arrival counter per (seq, kv head)
  float* out;
  uint32_t* arrive;
};

struct MergeArgs {
  const float* pm;
  const float* pl;
  const float* pacc;
  const float* pi;
  int n_cold_splits;
  int n_splits;
  int n_q_heads;
  int n_kv_heads;
  float* out;       // normalised output, or nullptr
  float* m_out;     // partial-state outputs (when out == nullptr)
  float* l_out;
  float* acc_out;
};

constexpr int kThreads = 256;
constexpr int kVOEnt = 2048;  // VALU decode: side-list entries staged in LDS per group

template <int GQ, bool IS_MAX>
__device__ __forceinline__ void block_reduce(float (&v)[GQ], float (*red)[GQ]) {
#pragma unroll
  for (int i = 0; i < GQ; ++i) v[i] = IS_MAX ? wave_max(v[i]) : wave_sum(v[i]);
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < GQ; ++i) red[threadIdx.x >> 6][i] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < GQ; ++i)
    v[i] = IS_MAX ? fmaxf(fmaxf(red[0][i], red[1][i]), fmaxf(red[2][i], red[3][i]))
                  : (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
  __syncthreads();
}

// Online-softmax update over the n scores in sc[i][0..n) (already scaled).
// On return sc[i][t] holds p_t (times the value norm when norms != nullptr).
template <int GQ>
__device__ __forceinline__ void softmax_update(float (*sc)[kThreads], int n, float (&m_run)[GQ],
                                               float (&l_run)[GQ], float (&acc0)[GQ],
                                               float (&acc1)[GQ], float (*red)[GQ],
                                               float norm_t) {
  const int t = threadIdx.x;
  float mx[GQ];
#pragma unroll
  for (int i = 0; i < GQ; ++i) mx[i] = (t < n) ? sc[i][t] : -INFINITY;
  block_reduce<GQ, true>(mx, red);
  float p[GQ], ps[GQ];
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    const float mn = fmaxf(m_run[i], mx[i]);
    const float corr = __expf(m_run[i] - mn);
    m_run[i] = mn;
    l_run[i] *= corr;
    acc0[i] *= corr;
    acc1[i] *= corr;
    p[i] = (t < n) ? __expf(sc[i][t] - mn) : 0.0f;
    ps[i] = p[i];
  }
  block_reduce<GQ, false>(ps, red);
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    l_run[i] += ps[i];
    if (t < n) sc[i][t] = p[i] * norm_t;
  }
  __syncthreads();
}

// A token's outlier corrections in the VALU decode: q_j * (val - dense_j) for
// its run of the token-sorted side-list oe (entries [lo, end) of its 32-token
// block hold it), found by binary search, added in list order.  Inlined at
// each call, so that a list staged in LDS is read with LDS loads.
template <int GQ, int D>
__device__ __forceinline__ void outlier_walk(const uint32_t* oe, int lo, int end, uint32_t first,
                                             const uint32_t* __restrict__ krow, int kb, int key_grid,
                                             const float* a_s, const float* mu_s,
                                             const float (*q_s)[D], float (&s)[GQ]) {
  int hi = end;
  while (lo < hi) {  // first entry of the run at or after (token, 0)
    const int mid = (lo + hi) >> 1;
    if ((oe[mid] & 0xFFFFu) < first) lo = mid + 1; else hi = mid;
  }
  for (int e = lo; e < end; ++e) {
    const uint32_t ent = oe[e];
    const uint32_t pos = ent & 0xFFFFu;
    if (pos >= first + D) break;
    const int j = (int)(pos - first);
    const uint32_t f = k_pair_index(krow, kb, j >> 1);
    const uint32_t c = (j & 1) ? k_code_odd(f, kb) : k_code_even(f, kb);
    const float delta = h2f((uint16_t)(ent >> 16)) - (a_s[j] * key_level(key_grid, c) + mu_s[j]);
#pragma unroll
    for (int i = 0; i < GQ; ++i) s[i] += q_s[i][j] * delta;
  }
}

// A token's dense key scores s[i] += w_i(pair) . levels(pair), pair by pair
// in channel order, by 32-channel chunks (KB words of the row each, read once
// per chunk): the 16 pairs of a chunk take their fields at fixed bit offsets
// (no per-pair switch on the key width or register-indexed row read).
template <int KB, int GQ, int D>
__device__ __forceinline__ void key_chunk_scores(const uint32_t (&rw)[D / 8], const float (*kl)[2],
                                                 const float2 (*w2)[GQ], float (&s)[GQ]) {
#pragma unroll 1
  for (int c = 0; c < D / 32; ++c) {
    uint32_t cw[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) cw[i] = rw[c * KB + i];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      uint32_t f;
      if constexpr (KB == 4) {
        f = (cw[p >> 2] >> (8 * (p & 3))) & 0xFFu;
      } else {
        constexpr int kF = 2 * KB;
        const int o = kF * p, w = o >> 5, sh = o & 31;
        uint32_t v = cw[w] >> sh;
        if (sh + kF > 32) v |= cw[w + 1] << (32 - sh);
        f = v & ((1u << kF) - 1u);
      }
      const float2 kk = *reinterpret_cast<const float2*>(&kl[f][0]);
#pragma unroll
      for (int i = 0; i < GQ; ++i) {
        const float2 ww = w2[c * 16 + p][i];
        s[i] = __builtin_fmaf(ww.y, kk.y, __builtin_fmaf(ww.x, kk.x, s[i]));
      }
    }
  }
}

// The VALU split kernel: pools the MFMA kernel does not take (head_dim 64 or
// 256, per-token value rows, a hot ring that is not whole 32-token blocks).
// Scores one token per thread; values one channel pair per thread over a
// slice of the tokens (D / 2 pairs x 512 / D slices).  Deterministic: every
// sum has a fixed order (a token's outlier corrections are added by the
// thread that scores it, in side-list order).
template <int GQ, int VB, int D>
__global__ __launch_bounds__(kThreads) void tqk_decode_split_valu(DecodeArgs a) {
  constexpr int VROW = D * VB / 8;
  constexpr int NP = D / 2;             // channel pairs
  constexpr int NQ = kThreads / NP;     // token slices of the value pass
  constexpr int TS = kThreads / NQ;     // tokens per slice (a group or hot split has <= 256)
  constexpr int NW = D / 64;            // waves that hold the per-channel bias terms (>= 1)
  static_assert(NP * NQ == kThreads && NW >= 1, "head_dim 64, 128 or 256");
  const int split = blockIdx.x + a.split_base, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const tqk_cache_desc& d = a.d;
  const int Hkv = d.n_kv_heads, Hq = d.n_q_heads, G = d.group_tokens, P = d.page_tokens;
  const int L = a.seq_lens[b];
  const int ng = n_groups_of(L, d.hot_window, G);
  const int n_cold = ng * G;
  const float sm = d.sm_scale;

  __shared__ float q_s[GQ][D];
  __shared__ float qr_s[GQ][D];  // q @ pi_t (PolarQuant keys' weights)
  // the group's key weights by channel pair and head: one 8-byte read gives a
  // head's two weights of a pair
  __shared__ float2 w2_s[NP][GQ];
  // the group's side-list, when it holds at most kVOEnt entries (the token
  // threads' searches and walks then read LDS, not memory)
  __shared__ uint32_t oe_s[kVOEnt];
  // the group's value code rows, staged by the token threads (one row each,
  // wide loads) for the value pass, whose threads walk the tokens of a slice
  // (not at 8 heads: the staging loads, live across the key loop, take all
  // 256 VGPRs of a wave there, and the value pass reads the rows itself)
  constexpr bool kStageV = GQ < 8;
  __shared__ __align__(16) uint32_t vrow_s[kStageV ? kThreads : 1][VROW / 4];
  static_assert(VROW % 4 == 0, "value rows of whole dwords");
  __shared__ float sc_s[GQ][kThreads];
  __shared__ float kl_s[256][2];
  __shared__ float vl_s[1 << (2 * VB)][2];
  __shared__ float red_s[4][GQ];
  __shared__ float a_s[D], mu_s[D];
  __shared__ float accr_s[NQ][GQ][D];

  // GQ is the kernel's power-of-two head count; the last GQ - gq heads are
  // zero-query padding whose states are never written
  const int gq = Hq / Hkv;
  const bool f32 = d.input_f32 != 0;  // fp32 query and hot ring
  for (int i = tid; i < GQ * D; i += kThreads) {
    const size_t qi = ((size_t)b * Hq + h * gq + i / D) * D + i % D;
    q_s[i / D][i % D] = (i / D >= gq) ? 0.f
                        : f32 ? static_cast<const float*>(a.q)[qi] : h2f(static_cast<const uint16_t*>(a.q)[qi]);
  }
  // key pair table: index of a channel pair (the code byte, or the 3-/2-bit
  // pair field) -> its two levels (PolarQuant keys: value centroids)
  const bool polar = a.d.key_grid == 2;
  {
    const uint32_t c0 = k_code_even((uint32_t)tid & 0xFFu, a.d.key_bits) & 15u;
    const uint32_t c1 = k_code_odd((uint32_t)tid & 0xFFu, a.d.key_bits) & 15u;
    const uint32_t cm = (1u << a.d.key_bits) - 1u;
    kl_s[tid][0] = polar ? a.p.vcent[c0 & cm] : key_level(a.d.key_grid, c0);
    kl_s[tid][1] = polar ? a.p.vcent[c1 & cm] : key_level(a.d.key_grid, c1);
  }
  // value pair table: field f of two channels' codes -> their two centroids
  if (tid < (1 << (2 * VB))) {
    vl_s[tid][0] = a.p.vcent[tid & ((1 << VB) - 1)];
    vl_s[tid][1] = a.p.vcent[tid >> VB];
  }

  if (polar) {
    __syncthreads();
    for (int i = tid; i < GQ * D; i += kThreads) {
      float x = 0.f;
      for (int dd = 0; dd < D; ++dd) x += q_s[i / D][dd] * a.p.pi_t[dd * D + i % D];
      qr_s[i / D][i % D] = x;
    }
  }

  float m_run[GQ], l_run[GQ], acc0[GQ], acc1[GQ];
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
    acc0[i] = 0.f;
    acc1[i] = 0.f;
  }
  __syncthreads();

  const int jp = tid % NP, tq = tid / NP;
  const int32_t* __restrict__ bt = a.p.block_table;

  if (split < a.n_cold_splits) {
    const int g0 = split * a.groups_per_split;
    const int g1 = min(ng, g0 + a.groups_per_split);
    // the group's slot and the token thread's page are read a group ahead
    // (their loads overlap the current group's instead of starting its chain;
    // not at 8 heads and head_dim 256, where the carried registers take all
    // 256 VGPRs)
    constexpr bool kAhead = !(GQ >= 8 && D >= 256);
    const int32_t* gt = a.p.group_table + (size_t)b * d.max_groups_per_seq;
    const int32_t* btb = bt + (size_t)b * d.max_pages_per_seq;
    int slot_nx = kAhead && g0 < g1 ? gt[g0] : 0;
    int phys_nx = kAhead && g0 < g1 && tid < G ? btb[(g0 * G + tid) / P] : 0;
    for (int g = g0; g < g1; ++g) {
      int slot, phys;
      if constexpr (kAhead) {
        slot = slot_nx;
        phys = phys_nx;
        if (g + 1 < g1) {
          slot_nx = gt[g + 1];
          if (tid < G) phys_nx = btb[((g + 1) * G + tid) / P];
        }
      } else {
        slot = gt[g];
        phys = 0;
      }
      const size_t mbase = ((size_t)slot * Hkv + h) * D;
      const size_t obase = (size_t)slot * Hkv + h;
      const int n_oe = d.outliers_per_channel > 0
                           ? min(a.p.ocount[obase * TQK_NOB + (G - 1) / TQK_OBLK], d.outlier_cap)
                           : 0;
      // (not at 8 heads and head_dim 256: a second inlined walk, or one over a
      // generic pointer, takes all 256 VGPRs there)
      const bool oe_lds = !(GQ >= 8 && D >= 256) && n_oe <= kVOEnt;
      if (oe_lds)
        for (int e = tid; e < n_oe; e += kThreads) oe_s[e] = a.p.oent[obase * d.outlier_cap + e];
      if (tid < D) {
        const float av = a.p.gscale[mbase + tid];
        const float mv = a.p.gmean[mbase + tid];
        a_s[tid] = av;
        mu_s[tid] = mv;
        float bias_part[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          reinterpret_cast<float*>(&w2_s[tid >> 1][i])[tid & 1] = (polar ? qr_s[i][tid] : q_s[i][tid]) * av;
          bias_part[i] = wave_sum(q_s[i][tid] * mv);
        }
        if ((tid & 63) == 0) {
#pragma unroll
          for (int i = 0; i < GQ; ++i) red_s[tid >> 6][i] = bias_part[i];
        }
      }
      __syncthreads();
      float bias[GQ];
#pragma unroll
      for (int i = 0; i < GQ; ++i) {
        bias[i] = red_s[0][i];
        if constexpr (NW == 2) bias[i] = red_s[0][i] + red_s[1][i];
        if constexpr (NW == 4) bias[i] = (red_s[0][i] + red_s[1][i]) + (red_s[2][i] + red_s[3][i]);
      }
      __syncthreads();

      // key scores, one token per thread: the dense part, then the token's
      // outlier corrections q_j * (val - dense_j) in side-list order (the
      // side-list is sorted by token; the cumulative counts at every 32nd
      // token bound the token's run, a binary search finds its start)
      float norm_t = 0.f;
      if (tid < G) {
        const size_t row = kAhead ? ((size_t)h * d.n_pages + phys) * P + (g * G + tid) % P
                                  : page_row(bt, d.max_pages_per_seq, b, g * G + tid, P, d.n_pages, h);
        const int kb = d.key_bits;
        const uint32_t* kr = reinterpret_cast<const uint32_t*>(a.p.kcodes + row * k_row_bytes(kb, D));
        // the token's key row: 16-byte loads where the row is whole 16-byte
        // pieces (a dword load per word touches each row's cache lines once
        // per word: one token per lane, rows a row apart)
        uint32_t rw[D / 8];
        const int kwords = k_row_bytes(kb, D) / 4;
        if ((kwords & 3) == 0) {
#pragma unroll
          for (int c4 = 0; c4 < D / 32; ++c4) {
            if (4 * c4 < kwords) {
              const uint4 x = reinterpret_cast<const uint4*>(kr)[c4];
              rw[4 * c4] = x.x;
              rw[4 * c4 + 1] = x.y;
              rw[4 * c4 + 2] = x.z;
              rw[4 * c4 + 3] = x.w;
            }
          }
        } else {
          for (int w2 = 0; w2 < kwords; ++w2) rw[w2] = kr[w2];
        }
        // the token's side-list run bounds (the cumulative counts of its
        // 32-token block and the one before) and norms, read beside the row
        // (where used, kAhead: again not at 8 heads and head_dim 256)
        const bool has_oe = d.outliers_per_channel > 0;
        const int* oc = a.p.ocount + obase * TQK_NOB;
        const int blk = tid / TQK_OBLK;
        const int oc_lo = kAhead && has_oe && blk > 0 ? oc[blk - 1] : 0;
        const int oc_hi = kAhead && has_oe ? oc[blk] : 0;
        const float vn = kAhead ? a.p.vnorm[row] : 0.f;
        // score = |k| * (q_rot . centroids)
        const float kn = kAhead ? (polar ? a.p.knorm[row] * sm : sm) : 0.f;
        // the token's value code row into LDS for the value pass (stored here,
        // before the score loop, so the row is not held in registers across it)
        if constexpr (kStageV) {
          const uint8_t* vsrc = a.p.vcodes + row * VROW;
          if constexpr (VROW % 16 == 0) {
#pragma unroll
            for (int c4 = 0; c4 < VROW / 16; ++c4)
              reinterpret_cast<uint4*>(&vrow_s[tid][0])[c4] = reinterpret_cast<const uint4*>(vsrc)[c4];
          } else {
#pragma unroll
            for (int w4 = 0; w4 < VROW / 4; ++w4) vrow_s[tid][w4] = reinterpret_cast<const uint32_t*>(vsrc)[w4];
          }
          asm volatile("" ::: "memory");
        }
        float s[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) s[i] = 0.f;
        if constexpr (GQ >= 8 && D >= 256) {
          // (pair by pair, not unrolled: a chunk's 16 pairs at 8 heads hoist
          // 128 weight pairs and take all 256 VGPRs)
#pragma unroll 1
          for (int jp2 = 0; jp2 < D / 2; ++jp2) {
            const uint32_t f = k_pair_index(rw, kb, jp2);
            const float2 kk = *reinterpret_cast<const float2*>(&kl_s[f][0]);
#pragma unroll
            for (int i = 0; i < GQ; ++i) {
              const float2 ww = w2_s[jp2][i];
              s[i] += ww.x * kk.x + ww.y * kk.y;
            }
          }
        } else if (kb == 4) {
          key_chunk_scores<4, GQ, D>(rw, kl_s, w2_s, s);
        } else if (kb == 3) {
          key_chunk_scores<3, GQ, D>(rw, kl_s, w2_s, s);
        } else {
          key_chunk_scores<2, GQ, D>(rw, kl_s, w2_s, s);
        }
#pragma unroll
        for (int i = 0; i < GQ; ++i) s[i] += bias[i];
        if (has_oe) {
          const int cap = d.outlier_cap;
          const int lo0 = min(kAhead ? oc_lo : (blk > 0 ? oc[blk - 1] : 0), cap);
          const int end = min(kAhead ? oc_hi : oc[blk], cap);
          const uint32_t first = (uint32_t)tid * D;
          if (oe_lds) {
            outlier_walk<GQ, D>(oe_s, lo0, end, first, kr, kb, a.d.key_grid, a_s, mu_s, q_s, s);
          } else {
            // (at 8 heads and head_dim 256 from the row's registers: the
            // row pointer held across the walk there takes all 256 VGPRs)
            if constexpr (GQ >= 8 && D >= 256)
              outlier_walk<GQ, D>(a.p.oent + obase * cap, lo0, end, first, rw, kb, a.d.key_grid, a_s,
                                  mu_s, q_s, s);
            else
              outlier_walk<GQ, D>(a.p.oent + obase * cap, lo0, end, first, kr, kb, a.d.key_grid, a_s,
                                  mu_s, q_s, s);
          }
        }
        const float kn2 = kAhead ? kn : (polar ? a.p.knorm[row] * sm : sm);
#pragma unroll
        for (int i = 0; i < GQ; ++i) sc_s[i][tid] = s[i] * kn2;
        norm_t = kAhead ? vn : a.p.vnorm[row];
      }
      __syncthreads();

      softmax_update<GQ>(sc_s, G, m_run, l_run, acc0, acc1, red_s, norm_t);

      // value accumulation in rotated code space: thread = (channel pair, token
      // slice), the code rows from LDS where staged above (softmax_update's
      // barriers order the stores before these reads), else from memory
      const int tend = min(G, tq * TS + TS);
      // (unrolled so that several tokens' loads are in flight; not at 8 heads
      // and head_dim 256, where it takes all 256 VGPRs)
      constexpr int kVU = kStageV ? 2 : (D >= 256 ? 1 : 4);
#pragma unroll kVU
      for (int tt = tq * TS; tt < tend; ++tt) {
        // the 2*VB-bit field of channels 2jp, 2jp + 1 in the token's bit stream
        const int bit = 2 * VB * jp, wd = bit >> 5, sh = bit & 31;
        uint32_t lo, hi;
        if constexpr (kStageV) {
          // (3-bit codes: the next word read for every lane, its bits shifted
          // out where the field does not cross; the last word's fields end
          // inside it, so its index is clamped to the row)
          lo = vrow_s[tt][wd];
          if constexpr (VB == 3) hi = vrow_s[tt][min(wd + 1, VROW / 4 - 1)];
          else hi = (sh + 2 * VB > 32) ? vrow_s[tt][wd + 1] : 0u;
        } else {
          const size_t row = page_row(bt, d.max_pages_per_seq, b, g * G + tt, P, d.n_pages, h);
          const uint32_t* vr = reinterpret_cast<const uint32_t*>(a.p.vcodes + row * VROW);
          lo = vr[wd];
          hi = (sh + 2 * VB > 32) ? vr[wd + 1] : 0u;
        }
        // (hi:lo) >> sh in one funnel shift
        const uint32_t f = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh) & ((1u << (2 * VB)) - 1u);
        const float c0 = vl_s[f][0], c1 = vl_s[f][1];
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          const float pp = sc_s[i][tt];
          acc0[i] += pp * c0;
          acc1[i] += pp * c1;
        }
      }
      __syncthreads();
    }
  } else {
    // hot window slice (fp16, or fp32 for input_f32)
    const int hs = split - a.n_cold_splits;
    const int t0 = n_cold + hs * a.hot_per_split;
    const int t1 = min(L, t0 + a.hot_per_split);
    if (t0 < t1) {
      const int n = t1 - t0;
      const int R = d.hot_ring;
      const size_t hbase = ((size_t)b * Hkv + h) * R;
      if (tid < n) {
        const size_t krow = (hbase + (t0 + tid) % R) * D;
        float s[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) s[i] = 0.f;
        if (f32) {
          const float2* kr = reinterpret_cast<const float2*>(static_cast<const float*>(a.p.hot_k) + krow);
#pragma unroll 4
          for (int jp2 = 0; jp2 < D / 2; ++jp2) {
            const float2 kk = kr[jp2];
#pragma unroll
            for (int i = 0; i < GQ; ++i) s[i] += q_s[i][2 * jp2] * kk.x + q_s[i][2 * jp2 + 1] * kk.y;
          }
        } else {
          const uint4* kr = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.p.hot_k) + krow);
#pragma unroll 4
          for (int c = 0; c < D / 8; ++c) {
            const uint4 w4 = kr[c];
            const uint32_t wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
              const float k0 = h2f((uint16_t)(wv[wi] & 0xFFFFu));
              const float k1 = h2f((uint16_t)(wv[wi] >> 16));
              const int j = c * 8 + wi * 2;
#pragma unroll
              for (int i = 0; i < GQ; ++i) s[i] += q_s[i][j] * k0 + q_s[i][j + 1] * k1;
            }
          }
        }
#pragma unroll
        for (int i = 0; i < GQ; ++i) sc_s[i][tid] = s[i] * sm;
      }
      __syncthreads();
      softmax_update<GQ>(sc_s, n, m_run, l_run, acc0, acc1, red_s, 1.0f);
      const int tend = min(n, tq * TS + TS);
      constexpr int kVUh = GQ >= 8 && D >= 256 ? 1 : 4;
#pragma unroll kVUh
      for (int tt = tq * TS; tt < tend; ++tt) {
        const size_t vrow = (hbase + (t0 + tt) % R) * D;
        float c0, c1;
        if (f32) {
          const float2 two = reinterpret_cast<const float2*>(static_cast<const float*>(a.p.hot_v) + vrow)[jp];
          c0 = two.x;
          c1 = two.y;
        } else {
          const uint32_t two = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.p.hot_v) + vrow)[jp];
          c0 = h2f((uint16_t)(two & 0xFFFFu));
          c1 = h2f((uint16_t)(two >> 16));
        }
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          const float pp = sc_s[i][tt];
          acc0[i] += pp * c0;
          acc1[i] += pp * c1;
        }
      }
    }
  }

  // combine the token slices and write the split's state
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    accr_s[tq][i][2 * jp] = acc0[i];
    accr_s[tq][i][2 * jp + 1] = acc1[i];
  }
  __syncthreads();
  const int ns = a.n_cold_splits + a.n_hot_splits;
  for (int x = tid; x < gq * D; x += kThreads) {
    const int i = x / D, j = x % D;
    float sq;
    if constexpr (NQ == 2) {
      sq = accr_s[0][i][j] + accr_s[1][i][j];
    } else if constexpr (NQ == 4) {
      sq = (accr_s[0][i][j] + accr_s[1][i][j]) + (accr_s[2][i][j] + accr_s[3][i][j]);
    } else {
      sq = ((accr_s[0][i][j] + accr_s[1][i][j]) + (accr_s[2][i][j] + accr_s[3][i][j])) +
           ((accr_s[4][i][j] + accr_s[5][i][j]) + (accr_s[6][i][j] + accr_s[7][i][j]));
    }
    a.pacc[(((size_t)b * Hq + h * gq + i) * ns + split) * D + j] = sq;
  }
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    if (tid == i && i < gq) {
      const size_t o = ((size_t)b * Hq + h * gq + i) * ns + split;
      a.pm[o] = m_run[i];
      a.pl[o] = l_run[i];
    }
  }
}


// ---------------------------------------------------------------------------
// MFMA split kernel (value codes in the tiled order, hot window ring % 32 == 0).
//
// 512 threads = 8 waves share one LDS code table.  A workgroup is either a
// coded split (its waves walk groups g0 + w, g0 + w + 8, ...) or the hot
// split of its (sequence, kv head) (waves walk 32-token blocks of the fp16
// window).  Every wave keeps an online-softmax state per query head and the
// workgroup folds the eight states into one partial at the end.
//
// Coded 32-token block (two 16-token tiles A, B):
//   QK^T  C[token][col] += A[token][ch] * B[ch][col]   (v_mfma_f32_16x16x32_f16)
//         A = NF4 level of the key code as fp16 hi + lo (two MFMAs),
//         B = q * nf4_scale as fp16 hi (cols 0..GQ-1) and lo (cols GQ..2GQ-1);
//         col h + col h+GQ is the full-precision score of query head h.
//   PV    O[row][ch] += P[row][token] * V[token][ch]   (one MFMA per 32 tokens)
//         P = softmax weight * value norm as fp16 hi (rows 0..7) or the fp16
//         residual (rows 8..15) of head row & (GQ - 1),
//         V = value centroid in fp16 (its rounding, <= 2^-12 relative, is
//         far inside the output tolerance; the weights need both halves).
// The QK^T accumulator layout (lane 16*lg + col holds tokens 4lg..4lg+3 of a
// tile) is the PV A-operand layout, so scores stay in registers; only blocks
// that hold outliers round-trip through a per-wave LDS block for the sparse
// q_j * (val - dense) corrections.  Key bytes become fp16 hi/lo operand pairs
// through a bank-replicated LDS table, value codes become fp16 centroids four
// tokens per lookup (LutGeom).  The next blocks' loads are issued before the
// current block is computed.
// ---------------------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x3_t __attribute__((ext_vector_type(3)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
// dword 3 of a raw buffer resource on gfx9 (32-bit data, no swizzle)
constexpr int kBufFlags = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufFlags);
}
typedef float floatx4_t __attribute__((ext_vector_type(4)));
union H8 {
  half8_t h;
  uint32_t u[4];
  uint4 v;
};

constexpr int kMWaves = 8;                 // waves per workgroup (two per SIMD)
constexpr int kMThreads = 64 * kMWaves;
constexpr int kMergeFast = 8;  // split counts merged with all partial loads issued up front
#ifndef TQK_COLD_BUFFERS
#define TQK_COLD_BUFFERS 3
#endif
constexpr int kColdBuf = TQK_COLD_BUFFERS;  // cold-stream register buffers (one more than blocks in flight)
constexpr int kMaxGPS = 128;     // groups per cold split of the MFMA kernel (metadata in LDS)
constexpr int kMetaInts = 32;    // per group: 16 tile rows, 8 outlier bounds, slot*Hkv+h
constexpr int kLutEntry = 256;   // bytes per table entry

// Code tables in LDS.
// Key table: entry e (a code byte of 4-bit keys, the 2^(2kb) pair fields of
// 3-/2-bit keys, value-code pairs for PolarQuant keys) holds {fp16 hi pair,
// fp16 lo pair} (8 bytes) of its two levels in kKeyCopies bank-spread copies:
// copy c at byte 8c of the entry's 256-byte row, so the bank of a lookup
// depends only on the lane's copy and random entries never share a bank.
// Value table: single fp16 centroids (the PV weights carry the fp16 hi/lo
// split instead), four tokens of one channel per lookup where possible:
//   3-bit values: the 12-bit field of four codes -> their four centroids
//     (8 bytes), 4096 entries, one copy (32 KiB) at offset 0; with 8 query
//     heads per kv head (whose outlier staging needs the LDS) the 6-bit
//     field of two codes -> two centroids (4 bytes) in 64 rows of 256 bytes;
//   2-bit values: a code byte (four codes) -> four centroids (8 bytes);
//   4-bit values: a code byte (two codes) -> two centroids (4 bytes);
//   byte tables take 256-byte rows like the key table.  With 4-bit keys the
//   key and value entries of byte e share row e (keys in its first 128
//   bytes, 16 copies; values in the second 128); otherwise a 2-/4-bit value
//   table fills its own 64 KiB of rows at offset 0.  The key rows follow
//   the value table.
template <int KB, int VB, int GQ>
struct LutGeom {
  static constexpr int kKeyEntries = KB == 4 ? 256 : 1 << (2 * KB);
  static constexpr bool kQuad12 = VB == 3 && GQ <= 4;
  static constexpr bool kPair6 = VB == 3 && GQ > 4;
  static constexpr bool kShared = KB == 4 && VB != 3;
  static constexpr int kKeyCopies = kShared ? 16 : 32;
  static constexpr int kValEntryBytes = VB == 4 || kPair6 ? 4 : 8;
  static constexpr int kValCopies = (kShared ? 128 : 256) / kValEntryBytes;
  static constexpr int kValBytes = kQuad12 ? 4096 * 8 : kPair6 ? 64 * 256 : (kShared ? 0 : 256 * 256);
  static constexpr uint32_t kKeyBase = kShared ? 0u : (uint32_t)kValBytes;
  static constexpr uint32_t kValOff = kShared ? 128u : 0u;  // value copy base inside a byte row
  static constexpr int kTableBytes = (int)kKeyBase + (kShared ? 256 : kKeyEntries) * kLutEntry;
  // at least 64 KiB: after the stream the area holds the waves' coded states
  // (8 x GQ x (D + 2) floats) and then Pi (D x D floats) for the merge
  static constexpr int kBytes = kTableBytes > 65536 ? kTableBytes : 65536;
};

__device__ __forceinline__ uint2 split_pair(float x0, float x1) {
  const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
  const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
  return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                    (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16));
}

// Workgroup barrier for LDS data only: this wave's LDS operations complete
// (lgkmcnt 0), then s_barrier.  Unlike __syncthreads it leaves the wave's
// global loads in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Orders LDS accesses of one wave across lanes.  A wave's LDS instructions
// execute in issue order, so program order is enough; this only stops the
// compiler from moving memory operations across the point (and, unlike a
// fence, does not wait for the wave's outstanding global loads).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// Cross-lane helpers without LDS traffic.
__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t x) { return __builtin_bit_cast(float, x); }
// max / sum over lanes {l, l^16, l^32, l^48}: the four token groups of a column
__device__ __forceinline__ float colgroup_max(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
  x = fmaxf(bitsf(a[0]), bitsf(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
  return fmaxf(bitsf(b[0]), bitsf(b[1]));
}
__device__ __forceinline__ float colgroup_sum(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(fbits(x), fbits(x), false, false);
  x = bitsf(a[0]) + bitsf(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
  return bitsf(b[0]) + bitsf(b[1]);
}
// value of lane (row-local) column c +/- N within the 16-lane row (DPP row rotate)
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return bitsf((uint32_t)__builtin_amdgcn_update_dpp(0, (int)fbits(x), 0x120 + N, 0xF, 0xF, false));
}

// LDS address of key-table entry (byte K of word x) for copy offset `off`
// (< 256): one v_perm_b32 -- byte 1 <- x.byte[K], byte 0 <- off, bytes 2,3 <- 0.
template <int K>
__device__ __forceinline__ uint32_t lut_addr_byte(uint32_t x, uint32_t off) {
  return __builtin_amdgcn_perm(x, off, 0x0C0C0000u | ((4u + K) << 8));
}

// 6-bit field M of a 96-bit value-code unit (3-bit codes), with 32-bit funnel
// shifts only: a 64-bit join of two words would be merged into one 8-byte read
// of the prefetch buffer, which then can no longer live in registers.
template <int W>
__device__ __forceinline__ uint32_t u4_word(const uint4& u) {
  return W == 0 ? u.x : W == 1 ? u.y : W == 2 ? u.z : u.w;
}
template <int M>
__device__ __forceinline__ uint32_t v3_field(const uint4& u) {
  constexpr int o = 6 * M, w = o / 32, sh = o % 32;
  if constexpr (sh + 6 <= 32) {
    return (u4_word<w>(u) >> sh) & 63u;
  } else {
    return __builtin_amdgcn_alignbit(u4_word<w + 1>(u), u4_word<w>(u), sh) & 63u;
  }
}

template <int VB>
struct ColdBlock {
  uint4 kA, kB;  // 16 key bytes of token c of tile A / B
  // value unit (lg, c) of tile A / B (12 bytes for 3-bit codes: .w unused).
  // Plain vector members, no arrays: an indexed private array here is moved
  // to LDS by the compiler, which then waits on every prefetch right away.
  uint4 uA, uB;
  float nv;        // value norm of token 16 * ((c >> 2) & 1) + 4lg + (c & 3)
  float kn;        // ... and its key norm (PolarQuant keys only)
};

// Per-wave online-softmax state for query head (c & (GQ - 1)) and the PV accumulators.
// Scores are kept in the log2 domain (q is pre-scaled by sm_scale * log2(e)).
// m is the head's running max (the same in every lane of its column) and
// mt = m + kLazyMax; l is this lane's share of the denominator (the weights of
// its own tokens), summed over the column when the state is read out.
struct WaveState {
  float m, mt, l;
  floatx4_t O[8];
};

__device__ __forceinline__ void reset_state(WaveState& st) {
  st.m = -INFINITY;
  st.mt = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) st.O[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
}

// Slack of the lazy running max, log2 units: weights p <= 4, so p * |v| stays
// finite in fp16 for value norms up to 16376
constexpr float kLazyMax = 2.0f;

// Online softmax over the 8 scores of this lane (tokens 4lg..4lg+3 of tiles A
// and B of column c).  Lazy running max: the heads keep their max, and the
// accumulators their scale, until one of the wave's scores exceeds its head's
// max by more than kLazyMax (a wave-uniform test on each lane's own scores,
// no cross-lane reduction); then every head takes its exact max and the state
// is rescaled.  (m, l, O) stays consistent for any m, so the softmax is the
// same.  Accumulator row r = 4lg + i belongs to head r & (GQ - 1), whose
// correction factor is read from that column with v_readlane.
template <int GQ>
__device__ __forceinline__ void softmax_block(WaveState& st, const float (&s)[8], float (&p)[8],
                                              int lg) {
  float bm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  bm = fmaxf(bm, fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
  if (__builtin_amdgcn_ballot_w64(bm > st.mt) != 0) {
    bm = colgroup_max(bm);
    const float mn = fmaxf(st.m, bm);
    const float corr = __builtin_amdgcn_exp2f(st.m - mn);
    st.m = mn;
    st.mt = mn + kLazyMax;
    st.l *= corr;
    // one factor per accumulator row, the rows as one vector (whole-vector
    // multiplies keep the accumulators in their registers)
    float cv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // no indexed array here: a lane-dependent pick from one would live in scratch
      const float c0 = bitsf((uint32_t)__builtin_amdgcn_readlane((int)fbits(corr), i & (GQ - 1)));
      float ci = c0;
      if constexpr (GQ > 4) {
        const float c1 = bitsf((uint32_t)__builtin_amdgcn_readlane((int)fbits(corr), 4 + i));
        ci = (lg & 1) ? c1 : c0;
      }
      cv[i] = ci;
    }
    const floatx4_t cvec = {cv[0], cv[1], cv[2], cv[3]};
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) st.O[nt] = st.O[nt] * cvec;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = __builtin_amdgcn_exp2f(s[i] - st.m);
    st.l += p[i];
  }
}

// Partial-state stores and the merge's loads of them.  The workgroups of one
// (seq, kv head) may run on different XCDs, each with its own L2: coherent
// (agent-scope) accesses make the partials visible to the merging workgroup
// without writing back or invalidating whole L2s.
__device__ __forceinline__ void st_agent(float* p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of one query head's ns split partials for channel j when there are
// more than kMergeFast: one online pass (running max M, the sums rescaled by
// e^{M_old - M_new} when a round raises it) over rounds of 2 * kMergeFast
// partials.  The loads of the next round are issued before the current one is
// combined (each round is a round trip to memory).  Partials at or past
// n_live are known to be empty (l = 0, which the pass skips anyway): they are
// not loaded.  Both merges (tqk_merge and the in-kernel one) use it, so they
// agree bit for bit whatever n_live they pass.
template <int D, class Load>
__device__ __forceinline__ void merge_chunked(Load ld, const float* pl, const float* pm,
                                              const float* pacc, size_t base, int ns, int n_live,
                                              int n_cold, int j, float& M, float& dn, float& cr,
                                              float& hh) {
  constexpr int C = 2 * kMergeFast;
  M = -INFINITY;
  dn = cr = hh = 0.f;
  const int nl = min(ns, n_live);
  if (nl <= 0) return;
  // (every load of a round is issued, at a clamped index, and its value
  // dropped past nl: the waits then stay exact)
  auto load_round = [&](int s0, float (&vl)[C], float (&vm)[C], float (&va)[C]) {
#pragma unroll
    for (int k = 0; k < C; ++k) {
      const bool ok = s0 + k < nl;
      const size_t si = base + (size_t)min(s0 + k, nl - 1);
      const float l = ld(pl + si), m = ld(pm + si), x = ld(pacc + si * D + j);
      vl[k] = ok ? l : 0.f;
      vm[k] = ok ? m : -INFINITY;
      va[k] = ok ? x : 0.f;
    }
  };
  auto combine_round = [&](int s0, const float (&vl)[C], const float (&vm)[C], const float (&va)[C]) {
    float Mc = M;
#pragma unroll
    for (int k = 0; k < C; ++k)
      if (vl[k] > 0.f) Mc = fmaxf(Mc, vm[k]);
    if (Mc > M) {
      const float f = __expf(M - Mc);  // 0 on the first round (the sums are 0)
      dn *= f;
      cr *= f;
      hh *= f;
      M = Mc;
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
      if (vl[k] > 0.f) {
        const float wt = __expf(vm[k] - M);
        dn += vl[k] * wt;
        const float x = va[k] * wt;
        if (s0 + k < n_cold) cr += x; else hh += x;
      }
    }
  };
  // two register sets, rounds in pairs: A holds rounds s0, B rounds s0 + C
  float al[C], am[C], aa[C], bl[C], bm[C], ba[C];
  load_round(0, al, am, aa);
  for (int s0 = 0; s0 < nl; s0 += 2 * C) {
    if (s0 + C < nl) load_round(s0 + C, bl, bm, ba);
    combine_round(s0, al, am, aa);
    if (s0 + C >= nl) break;
    if (s0 + 2 * C < nl) load_round(s0 + 2 * C, al, am, aa);
    combine_round(s0 + C, bl, bm, ba);
  }
}

// Lane I of each 16-lane row, broadcast to the row (DPP row_newbcast).
template <int I>
__device__ __forceinline__ float row_bcast(float x) {
  return bitsf((uint32_t)__builtin_amdgcn_update_dpp(0, (int)fbits(x), 0x150 + I, 0xF, 0xF, false));
}

template <int K>
struct IntC {
  static constexpr int value = K;
};

// fp16 pair (RNE) of two floats in one dword, and the fp32 value of a half
__device__ __forceinline__ uint32_t pk_f16(float x, float y) {
  typedef float float2_t __attribute__((ext_vector_type(2)));
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t hv = __builtin_convertvector((float2_t){x, y}, half2_t);
  return __builtin_bit_cast(uint32_t, hv);
}
__device__ __forceinline__ float lo_f16(uint32_t pk) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(pk & 0xFFFFu)); }
__device__ __forceinline__ float hi_f16(uint32_t pk) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(pk >> 16)); }

// MFMA operand quad [x0 x1 x0 x1 x2 x3 x2 x3]: each value twice, so that it
// meets both the fp16 hi and the fp16 lo k-slot of the other operand.  The
// halves are fp16(x) (lo_sel = 0) or the fp16 residual x - fp16(x) (lo_sel = 1).
// Used for the PV weights (x = weights of tokens 4lg..4lg+3 of a tile) and for
// the QK^T weights (x = q * nf4_scale of four channels).
__device__ __forceinline__ H8 dup_quad(float x0, float x1, float x2, float x3, float lo_sel) {
  const uint32_t h01 = pk_f16(x0, x1), h23 = pk_f16(x2, x3);
  const uint32_t v01 = pk_f16(fmaf(-lo_sel, lo_f16(h01), x0), fmaf(-lo_sel, hi_f16(h01), x1));
  const uint32_t v23 = pk_f16(fmaf(-lo_sel, lo_f16(h23), x2), fmaf(-lo_sel, hi_f16(h23), x3));
  H8 r;
  r.u[0] = v01;
  r.u[1] = v01;
  r.u[2] = v23;
  r.u[3] = v23;
  return r;
}

// Eight floats as fp16 (lo_sel = 0) or as the fp16 residual x - fp16(x)
// (lo_sel = 1), in pairs: the PV weight operand.
__device__ __forceinline__ H8 split8(float x0, float x1, float x2, float x3, float x4, float x5,
                                     float x6, float x7, float lo_sel) {
  auto pair = [&](float a, float b) {
    const uint32_t h = pk_f16(a, b);
    return pk_f16(fmaf(-lo_sel, lo_f16(h), a), fmaf(-lo_sel, hi_f16(h), b));
  };
  H8 r;
  r.u[0] = pair(x0, x1);
  r.u[1] = pair(x2, x3);
  r.u[2] = pair(x4, x5);
  r.u[3] = pair(x6, x7);
  return r;
}

// Tokens per outlier-correction segment: a whole 256-token group, or half of
// one with 8 query heads per kv head (so that the per-wave buffers of
// GQ x kSegTokens floats fit the LDS beside the code tables).
template <int GQ>
constexpr int kSegTokens = GQ > 4 ? 128 : 256;

// PK: PolarQuant keys (key_grid 2, KB == VB): the key table holds centroids,
// the QK^T weights are the rotated query, and every score is scaled by its
// token's key norm
template <int GQ, int VB, int KB, bool PK>
__global__ __launch_bounds__(kMThreads, 1) void tqk_decode_split_mfma(DecodeArgs a) {
  constexpr int D = TQK_D;
  constexpr int VROW = D * VB / 8;
  constexpr int KROW = D * KB / 8;  // key code bytes per token (tqk_common.h layout)
  constexpr int UNIT = VROW / 4;
  // 1-D grid over (split, kv head, seq), split fastest.  Every workgroup
  // streams the coded groups of its split and then its share of the fp16 hot
  // window, and writes two partials: coded (index split) and hot (index
  // n_cold_splits + split); a separate round of hot workgroups would only
  // start as coded ones finish
  int split, h, b;
  {
    const int Hkv_ = a.d.n_kv_heads, ncs = a.n_cold_splits;
    int item = blockIdx.x;
    split = item % ncs;
    item /= ncs;
    h = item % Hkv_;
    b = item / Hkv_;
    // Batches: take the (seq, split) items longest first -- most coded groups
    // first, ties in index order -- so that in a ragged batch the long items
    // start in the first rounds of workgroups and the short ones fill in
    // behind them.  Every workgroup ranks the same items the same way, so
    // (rank, kv head) <-> blockIdx.x is a bijection.  More items than the
    // workgroup has threads keep the plain order.
    const int n_items = a.batch * ncs;
    if (a.reorder && a.batch > 1 && n_items <= kMWaves * 64) {
      __shared__ int work_s[kMWaves * 64];
      __shared__ int pick_s;
      const int t = threadIdx.x;
      int wk = 0;
      if (t < n_items) {
        const int ng_t = n_groups_of(a.seq_lens[t / ncs], a.d.hot_window, a.d.group_tokens);
        wk = min(max(ng_t - (t % ncs) * a.groups_per_split, 0), a.groups_per_split);
        work_s[t] = wk;
      }
      __syncthreads();
      const int want = blockIdx.x / Hkv_;
      if (t < n_items) {
        int rank = 0;
        for (int j = 0; j < n_items; ++j) {
          const int wj = work_s[j];
          rank += (wj > wk) | ((wj == wk) & (j < t));
        }
        if (rank == want) pick_s = t;
      }
      __syncthreads();
      const int it = pick_s;
      b = it / ncs;
      split = it % ncs;
      h = blockIdx.x % Hkv_;
    }
  }
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lg = lane >> 4, c = lane & 15;
  const tqk_cache_desc& d = a.d;
  const int Hkv = d.n_kv_heads, Hq = d.n_q_heads, G = d.group_tokens, P = d.page_tokens;
  const int L = a.seq_lens[b];
  // scores in the log2 domain: q * sm_scale * log2(e), softmax with exp2
  const float qscale = d.sm_scale * 1.4426950408889634f;

  __shared__ __align__(16) uint8_t lut[LutGeom<KB, VB, GQ>::kBytes];
  // the area's later uses: the coded wave states of the fold, Pi in the merge
  static_assert(LutGeom<KB, VB, GQ>::kBytes >= (int)sizeof(float) * kMWaves * GQ * (D + 2), "fold area");
  static_assert(LutGeom<KB, VB, GQ>::kBytes >= (int)sizeof(float) * D * D, "Pi area");
  // raw fp16 q, channel-major: the outlier corrections' gathers
  __shared__ __align__(16) uint16_t qc_s[D][GQ];
  __shared__ __align__(16) uint16_t qf_s[GQ][D];        // raw fp16 q, head-major (hot-window operand)
  // scaled q, head-major; rows padded by 4 banks so that the head rows read by
  // one lane group fall in different banks
  __shared__ __align__(16) float q_h_s[GQ][D + 4];
  // (nf4_scale[128], nf4_mean[128]) of the group a wave starts next
  __shared__ __align__(16) float gsm_s[kMWaves][2 * D];
  // per wave: the QK^T initial value of every token of its current group
  // segment (kSegTokens tokens) and head, mean bias plus outlier corrections
  // ([head][token])
  constexpr int kCT = kSegTokens<GQ>;
  constexpr int kRow = kCT;
  __shared__ __align__(16) float corr_s[kMWaves][GQ][kRow];
  // per wave and head: the lo columns' initial value, the group's mean bias
  // q . mean (four copies: one tile's accumulator)
  __shared__ __align__(16) float bias_s[kMWaves][GQ][4];
  // NF4 levels [0, 16) and value centroids [16, 16 + 2^vb) in lanes of every
  // wave, for the table fill (loaded first: the fill waits for them only)
  // (both loads unconditional and the pick by bit masks: a select the
  // compiler turns into branches would sink each load into its own)
  const uint32_t cen = fbits(a.p.vcent[(lane & 15) & ((1 << VB) - 1)]);
  const uint32_t nf4 = fbits(kNF4[lane & 15]);
  const uint32_t unif = fbits((float)(lane & 15));
  const bool is_cen = lane < 16 ? PK && lane < (1 << KB) : lane < 16 + (1 << VB);
  const bool is_key = lane < 16 && !PK;
  const uint32_t mk_c = is_cen ? ~0u : 0u, mk_k = is_key ? ~0u : 0u, mk_u = a.d.key_grid ? ~0u : 0u;
  const float lvl = bitsf((cen & mk_c) | (((nf4 & ~mk_u) | (unif & mk_u)) & mk_k));
  // Metadata of the split's groups, read once here so the block stream issues
  // nothing but block loads: [0, 16) first row of each 16-token tile
  // (relative to this head's page region), [16, 24) cumulative outlier
  // bounds, [24] slot * Hkv + h.  Only rows below the split's group count
  // are read (the waves' groups); the rows of the last row block past it are
  // zero, later ones are not written.  Thread tid fills field mf of rows
  // mrow(r).  The set-up is
  // two memory round trips: the group slots and tile rows of every row are
  // loaded before the sequence length is known (indices clamped to the
  // tables' rows; rows past the split's groups are dropped once it is),
  // together with the length, the levels and q; the code tables are filled
  // while they are in flight; then the outlier bounds of the split's groups
  // are loaded by slot.
  __shared__ int meta_s[kMaxGPS][kMetaInts];
  constexpr int kMetaRows = kMThreads / kMetaInts;
  constexpr int kMetaIt = kMaxGPS / kMetaRows;
  static_assert(kMThreads % kMetaInts == 0 && kMaxGPS % kMetaRows == 0, "metadata rows");
  static_assert(kMetaRows == 2 * kMWaves && kMetaInts == 32, "two metadata rows per wave and block");
  const int mf = tid % kMetaInts;
  // row of block r filled by this thread: wave w fills rows w + 8k, the rows
  // of the groups it streams when splits are shared out in whole groups
  auto mrow = [&](int r) { return w + kMWaves * (2 * r + (lane >> 5)); };
  const int gbeg_m = split * a.groups_per_split;
  // (every load below is issued by every thread, at an index inside its
  // table, and its value selected afterwards: a load inside a branch would
  // be waited for where the branches join)
  // (tables without rows: entry 0 of seq_lens stands in, never used)
  const bool tables = d.max_groups_per_seq > 0 && d.max_pages_per_seq > 0;
  const int mg = max(d.max_groups_per_seq, 1), mp = max(d.max_pages_per_seq, 1);
  const int32_t* const gtab = tables ? a.p.group_table : a.seq_lens;
  const int32_t* const btab = tables ? a.p.block_table : a.seq_lens;
  // Only the row blocks a split of groups_per_split groups can use are
  // loaded; the others load from an empty buffer (zeros, no memory access),
  // so that every thread issues the same loads and the fill below waits for
  // the levels alone.
  const int n_it = (a.groups_per_split + kMetaRows - 1) / kMetaRows;
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(gtab, tables ? 4u * (uint32_t)a.batch * (uint32_t)mg : 4u);
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(btab, tables ? 4u * (uint32_t)a.batch * (uint32_t)mp : 4u);
  const __amdgpu_buffer_rsrc_t rnone = buf_rsrc(gtab, 0u);
  int slot_r[kMetaIt], phys_r[kMetaIt];
#pragma unroll
  for (int r = 0; r < kMetaIt; ++r) {
    const int g = min(gbeg_m + mrow(r), mg - 1);
    const int t = g * G + 16 * (mf & 15);
    const uint32_t gi = tables ? (uint32_t)b * (uint32_t)mg + (uint32_t)g : 0u;
    const uint32_t bi = tables ? (uint32_t)b * (uint32_t)mp + (uint32_t)min(t / P, mp - 1) : 0u;
    slot_r[r] = (int)__builtin_amdgcn_raw_buffer_load_b32(r < n_it ? rg : rnone, (int)(4u * gi), 0, 0);
    phys_r[r] = (int)__builtin_amdgcn_raw_buffer_load_b32(r < n_it ? rb : rnone, (int)(4u * bi), 0, 0);
  }
  // GQ is the kernel's power-of-two head count; the last GQ - gq heads are
  // zero-query padding (their columns score 0) whose states are never written
  const int gq = Hq / Hkv;
  constexpr int kQIt = (GQ * D + kMThreads - 1) / kMThreads;
  uint32_t qraw[kQIt];
#pragma unroll
  for (int r = 0; r < kQIt; ++r) {
    const int i = min(tid + r * kMThreads, GQ * D - 1);
    const int hi = min(i / D, gq - 1);
    const uint32_t x = static_cast<const uint16_t*>(a.q)[((size_t)b * Hq + h * gq + hi) * D + i % D];
    qraw[r] = i / D < gq ? x : 0u;
  }
  const int ng = n_groups_of(L, d.hot_window, G);
  // the levels go through the wave's own stats slot (free until the stream
  // starts): a wave-local exchange, no workgroup barrier in front of the fill
  if (lane < 32) gsm_s[w][lane] = lvl;
  wave_sync();
  {
    // key unit u (8 bytes): entry u / copies, copy u % copies; consecutive
    // lanes write consecutive units; levels come from LDS, so the fill issues
    // no memory loads
    const float* lv = &gsm_s[w][0];
    using LG = LutGeom<KB, VB, GQ>;
    constexpr int NC = LG::kKeyCopies;
    constexpr int NK = LG::kKeyEntries;
    for (int u = tid; u < NK * NC; u += kMThreads) {
      const uint32_t e = (uint32_t)(u / NC);
      *reinterpret_cast<uint2*>(lut + LG::kKeyBase + e * kLutEntry + (uint32_t)(u % NC) * 8u) =
          split_pair(lv[k_code_even(e, KB)], lv[k_code_odd(e, KB)]);
    }
    const float* cv = lv + 16;  // value centroids
    if constexpr (LG::kQuad12) {
      // entry e: centroids of codes e & 7, e >> 3 & 7, e >> 6 & 7, e >> 9
      for (uint32_t e = tid; e < 4096u; e += kMThreads)
        *reinterpret_cast<uint2*>(lut + 8u * e) =
            make_uint2(pk_f16(cv[e & 7u], cv[(e >> 3) & 7u]), pk_f16(cv[(e >> 6) & 7u], cv[e >> 9]));
    } else {
      constexpr int NVC = LG::kValCopies, EB = LG::kValEntryBytes;
      constexpr int NE = LG::kPair6 ? 64 : 256;
      for (int u = tid; u < NE * NVC; u += kMThreads) {
        const uint32_t e = (uint32_t)(u / NVC), off = e * kLutEntry + LG::kValOff + (uint32_t)(u % NVC) * EB;
        if constexpr (LG::kPair6) {
          *reinterpret_cast<uint32_t*>(lut + off) = pk_f16(cv[e & 7u], cv[e >> 3]);
        } else if constexpr (VB == 4) {
          *reinterpret_cast<uint32_t*>(lut + off) = pk_f16(cv[e & 15u], cv[e >> 4]);
        } else {
          *reinterpret_cast<uint2*>(lut + off) =
              make_uint2(pk_f16(cv[e & 3u], cv[(e >> 2) & 3u]), pk_f16(cv[(e >> 4) & 3u], cv[e >> 6]));
        }
      }
    }
  }
  {
    // the outlier bounds of the split's groups by slot, then the rows
    const int gcnt = max(0, min(ng, gbeg_m + a.groups_per_split) - gbeg_m);
    int oc_r[kMetaIt];
#pragma unroll
    for (int r = 0; r < kMetaIt; ++r) {
      oc_r[r] = 0;
      if (r >= n_it) continue;
      const bool in = mrow(r) < gcnt;
      const uint32_t obase = (uint32_t)slot_r[r] * (uint32_t)Hkv + (uint32_t)h;
      // (entry 0 for the rows and fields that take no bound)
      const size_t oi = in && mf >= 16 && mf < 16 + TQK_NOB ? (size_t)obase * TQK_NOB + (mf - 16) : 0;
      oc_r[r] = a.p.ocount[oi];
    }
#pragma unroll
    for (int r = 0; r < kMetaIt; ++r) {
      if (r >= n_it) continue;
      const int jg = mrow(r);
      const int g = min(gbeg_m + jg, mg - 1);
      const int t = g * G + 16 * (mf & 15);
      const uint32_t obase = (uint32_t)slot_r[r] * (uint32_t)Hkv + (uint32_t)h;
      int v = 0;
      if (mf < G / 16)  // first row of tile mf, phys P + t % P inside head h's region
        v = (int)((uint32_t)phys_r[r] * (uint32_t)P + (uint32_t)(t % P));
      else if (mf >= 16 && mf < 16 + TQK_NOB)
        v = min(oc_r[r], d.outlier_cap);
      else if (mf == 16 + TQK_NOB)
        v = (int)obase;
      meta_s[jg][mf] = jg < gcnt ? v : 0;
    }
  }
#pragma unroll
  for (int r = 0; r < kQIt; ++r) {
    const int i = tid + r * kMThreads;
    if (i < GQ * D) {
      qc_s[i % D][i / D] = (uint16_t)qraw[r];
      qf_s[i / D][i % D] = (uint16_t)qraw[r];
      q_h_s[i / D][i % D] = h2f((uint16_t)qraw[r]) * qscale;
    }
  }
  // (the set-up's workgroup barrier is the stream's lds_barrier below: until
  // it a wave reads only its own metadata rows)
  if constexpr (PK) {
    __syncthreads();
    // the coded keys' weights: the rotated query q @ pi_t (scaled), from the raw q
    float qrot[(GQ * D + kMThreads - 1) / kMThreads];
#pragma unroll
    for (int r = 0; r < (GQ * D + kMThreads - 1) / kMThreads; ++r) {
      const int i = tid + r * kMThreads;
      float x = 0.f;
      if (i < GQ * D)
        for (int dd = 0; dd < D; ++dd) x += h2f(qf_s[i / D][dd]) * a.p.pi_t[dd * D + i % D];
      qrot[r] = x * qscale;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < (GQ * D + kMThreads - 1) / kMThreads; ++r) {
      const int i = tid + r * kMThreads;
      if (i < GQ * D) q_h_s[i / D][i % D] = qrot[r];
    }
    __syncthreads();
  }

  // Columns of the score tiles and rows of the PV tiles: c < 8 carry fp16 hi
  // parts, c >= 8 the fp16 lo parts, of head c & (GQ - 1) (heads repeat when
  // GQ < 8; only rows with (c & 7) < GQ are read out at the end).
  const int hq = c & (GQ - 1);
  const bool is_hi = c < 8;
  const float lo_sel = is_hi ? 0.f : 1.f;
  // hi column + lo column of the same head (lane c and c ^ 8 of a row)
  auto pair_sum = [&](float x) { return x + row_ror<8>(x); };
  WaveState st;
  reset_state(st);

  {
    constexpr int NC = LutGeom<KB, VB, GQ>::kKeyCopies;
    const uint32_t koff = (uint32_t)(lane % NC) * 8u;
    // (byte value tables) this lane's value copy inside a row
    const uint32_t voff = LutGeom<KB, VB, GQ>::kValOff +
                          (uint32_t)(lane % LutGeom<KB, VB, GQ>::kValCopies) * LutGeom<KB, VB, GQ>::kValEntryBytes;
    const uint8_t* __restrict__ klut = lut + LutGeom<KB, VB, GQ>::kKeyBase;
    const int cap = d.outlier_cap;
    // the side-list base (a valid pointer even without a side-list)
    const uint32_t* __restrict__ oent_all = cap > 0 ? a.p.oent : reinterpret_cast<const uint32_t*>(a.p.ocount);
    // This wave streams T blocks, block after block: the split's groups wu,
    // wu + 8, ... whole (meta_s rows g0 + gstep * j), or, for splits of fewer
    // groups than waves, wave_blocks consecutive blocks of the split starting
    // at block kb0 of its first group.
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int gbeg = split * a.groups_per_split;
    const int gcnt = max(0, min(ng, gbeg + a.groups_per_split) - gbeg);
    const int nblk = G / 32;
    int g0, gstep, kb0, nw, T;
    if (a.wave_blocks > 0) {
      const int b0 = wu * a.wave_blocks;
      T = max(0, min(a.wave_blocks, gcnt * nblk - b0));
      g0 = b0 / nblk;
      kb0 = b0 % nblk;
      gstep = 1;
      nw = T > 0 ? (kb0 + T + nblk - 1) / nblk : 0;
    } else {
      g0 = wu;
      kb0 = 0;
      gstep = kMWaves;
      nw = wu < gcnt ? (gcnt - wu + kMWaves - 1) / kMWaves : 0;
      T = nw * nblk;
    }
    // per-lane parts of the block addresses (the row parts are wave-uniform)
    // (the lane's token row c, its 32-channel chunk lg)
    const uint32_t koffL = (uint32_t)c * KROW + (uint32_t)(KROW / 4) * (uint32_t)lg;
    const uint32_t uoffL = (uint32_t)(16 * lg + c) * UNIT;
    const int ntl = 4 * lg + (c & 3);  // token (of tile A if c & 4 == 0, else B) whose norm this lane reads
    auto meta = [&](int j, int f) { return __builtin_amdgcn_readfirstlane(meta_s[g0 + gstep * j][f]); };
    // the metadata of the wave group being loaded (jl below), field f in lane
    // f: the block loads read it with v_readlane, with no LDS round trip per block
    int mv = 0;
    auto load_meta = [&](int j) {
      mv = (lane < kMetaInts && nw > 0) ? meta_s[g0 + gstep * min(j, nw - 1)][lane] : 0;
    };
    auto meta_l = [&](int f) { return __builtin_amdgcn_readlane(mv, f); };
    // buffer resources of this head's page regions (32-bit offsets:
    // mfma_path() bounds a head's region below 4 GiB)
    const uint32_t hrows = (uint32_t)d.n_pages * (uint32_t)P;
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(a.p.kcodes + (size_t)h * hrows * KROW, hrows * KROW);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(a.p.vcodes + (size_t)h * hrows * VROW, hrows * VROW);
    const __amdgpu_buffer_rsrc_t rn = buf_rsrc(a.p.vnorm + (size_t)h * hrows, hrows * 4u);
    const __amdgpu_buffer_rsrc_t rkn = buf_rsrc(PK ? a.p.knorm + (size_t)h * hrows : a.p.vnorm, PK ? hrows * 4u : 0u);

    // Every step issues the same block loads (past the end: the last block
    // again, already in L2), so the waits on the oldest buffer stay exact.
    int jl = 0, kbl = kb0, nl = 0;  // next block to load: wave group jl, block kbl, stream index nl
    // whole-group shares: the wave's rows are its own (filled by it above)
    const bool own_rows = a.wave_blocks == 0;
    if (own_rows) load_meta(0);
    auto load_next = [&](ColdBlock<VB>& cb) {
      // rows of the two tiles in this head's region (wave-uniform: SGPR offsets)
      const uint32_t rowA = (uint32_t)meta_l(2 * kbl);
      const uint32_t rowB = (uint32_t)meta_l(2 * kbl + 1);
      if constexpr (KB == 4) {
        const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)koffL, (int)(rowA * KROW), 0);
        const u32x4_t y = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)koffL, (int)(rowB * KROW), 0);
        cb.kA = make_uint4(x.x, x.y, x.z, x.w);
        cb.kB = make_uint4(y.x, y.y, y.z, y.w);
      } else if constexpr (KB == 3) {
        const u32x3_t x = __builtin_amdgcn_raw_buffer_load_b96(rk, (int)koffL, (int)(rowA * KROW), 0);
        const u32x3_t y = __builtin_amdgcn_raw_buffer_load_b96(rk, (int)koffL, (int)(rowB * KROW), 0);
        cb.kA = make_uint4(x.x, x.y, x.z, 0u);
        cb.kB = make_uint4(y.x, y.y, y.z, 0u);
      } else {
        const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(rk, (int)koffL, (int)(rowA * KROW), 0);
        const u32x2_t y = __builtin_amdgcn_raw_buffer_load_b64(rk, (int)koffL, (int)(rowB * KROW), 0);
        cb.kA = make_uint4(x.x, x.y, 0u, 0u);
        cb.kB = make_uint4(y.x, y.y, 0u, 0u);
      }
      if constexpr (VB == 2) {
        const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(rv, (int)uoffL, (int)(rowA * VROW), 0);
        const u32x2_t y = __builtin_amdgcn_raw_buffer_load_b64(rv, (int)uoffL, (int)(rowB * VROW), 0);
        cb.uA = make_uint4(x.x, x.y, 0u, 0u);
        cb.uB = make_uint4(y.x, y.y, 0u, 0u);
      } else if constexpr (VB == 3) {
        const u32x3_t x = __builtin_amdgcn_raw_buffer_load_b96(rv, (int)uoffL, (int)(rowA * VROW), 0);
        const u32x3_t y = __builtin_amdgcn_raw_buffer_load_b96(rv, (int)uoffL, (int)(rowB * VROW), 0);
        cb.uA = make_uint4(x.x, x.y, x.z, 0u);
        cb.uB = make_uint4(y.x, y.y, y.z, 0u);
      } else {
        const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)uoffL, (int)(rowA * VROW), 0);
        const u32x4_t y = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)uoffL, (int)(rowB * VROW), 0);
        cb.uA = make_uint4(x.x, x.y, x.z, x.w);
        cb.uB = make_uint4(y.x, y.y, y.z, y.w);
      }
      // (the lane's own tile row: with 16-token pages tile B may sit on a page
      // below tile A's, so the row is picked per lane, not offset from rowA)
      cb.nv = bitsf(__builtin_amdgcn_raw_buffer_load_b32(
          rn, (int)(4u * (((c & 4) ? rowB : rowA) + (uint32_t)ntl)), 0, 0));
      if constexpr (PK)
        cb.kn = bitsf(__builtin_amdgcn_raw_buffer_load_b32(
            rkn, (int)(4u * (((c & 4) ? rowB : rowA) + (uint32_t)ntl)), 0, 0));
      if (nl + 1 < T) {
        ++nl;
        if (++kbl == nblk) {
          kbl = 0;
          ++jl;
          load_meta(jl);
        }
      }
    };

    // (nf4_scale, nf4_mean) of channels 2*lane, 2*lane + 1 of a wave group,
    // staged through registers into the wave's LDS slot: every step loads the
    // stats of the group of the block it prefetches (before the block loads,
    // unconditionally, so the loads are never sunk to their use) and the next
    // step writes them, before that group can start.  One slot suffices: a
    // group's stats are read only at its start (weights, bias, corrections),
    // and a group's first block is computed a step after its stats arrive.
    float2 pend_s, pend_m;  // stats loaded by the previous step
    // (obase: slot * Hkv + h of the group)
    auto load_group_stats = [&](int obase) {
      const size_t mb = (size_t)D * (uint32_t)obase;
      const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(buf_rsrc(a.p.gscale + mb, 4u * D), 8 * lane, 0, 0);
      const u32x2_t y = __builtin_amdgcn_raw_buffer_load_b64(buf_rsrc(a.p.gmean + mb, 4u * D), 8 * lane, 0, 0);
      pend_s = make_float2(bitsf(x.x), bitsf(x.y));
      pend_m = make_float2(bitsf(y.x), bitsf(y.y));
    };
    auto store_group_stats = [&]() {
      *reinterpret_cast<float2*>(&gsm_s[w][2 * lane]) = pend_s;
      *reinterpret_cast<float2*>(&gsm_s[w][D + 2 * lane]) = pend_m;
    };
    // QK^T: C[token][col] = sum_k A[token][k] * B[k][col] over k-slots that
    // pair each channel's fp16 hi and lo NF4 level with the same weight.
    // MFMA m takes key bytes 2m, 2m+1 of the lane's 16 (channels ch0..ch3 =
    // 32lg + 4m + 0..3): A k-slots [hi ch0, hi ch1, lo ch0, lo ch1, hi ch2,
    // hi ch3, lo ch2, lo ch3] are two table rows read straight into the
    // operand, B = [w0 w1 w0 w1 w2 w3 w2 w3] with w = q * nf4_scale of the
    // column's head as fp16 hi (c < 8) or lo (c >= 8).  Column c plus column
    // c ^ 8 is the fp32 score.  The hi columns start from the group's per-token
    // initial values (mean bias plus the token's outlier corrections, built
    // once per group in corr_s); the lo columns start from zero.
    H8 Bw[8];
    float bias_h;  // q . mean of head hq (the lo columns' initial value)
    // Start of wave group j: weights and mean bias from the wave's stats slot.
    auto begin_group = [&]() {
      const float* gs = &gsm_s[w][0];
      float biasp = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int ch = 32 * lg + 4 * m;
        const float4 q4 = *reinterpret_cast<const float4*>(&q_h_s[hq][ch]);
        const float4 s4 = *reinterpret_cast<const float4*>(&gs[ch]);
        const float4 m4 = *reinterpret_cast<const float4*>(&gs[D + ch]);
        biasp += q4.x * m4.x + q4.y * m4.y + q4.z * m4.z + q4.w * m4.w;
        Bw[m] = dup_quad(q4.x * s4.x, q4.y * s4.y, q4.z * s4.z, q4.w * s4.w, lo_sel);
      }
      bias_h = colgroup_sum(biasp);
      // lanes c < GQ of lane group 0: the bias of head c, four copies
      if (lane < GQ) *reinterpret_cast<float4*>(&bias_s[w][lane][0]) = make_float4(bias_h, bias_h, bias_h, bias_h);
    };

    // ---- sparse outliers, once per segment of kCT tokens of a group: the
    // score of token t for head h gains q_h[j] * (val - mean_j) for every
    // side-list entry (t, j, val) (the stored code of an outlier is the NF4
    // zero level, so the dense pass gave exactly mean_j there, inside the
    // bias).  The wave turns the segment's stretch of the token-sorted
    // side-list into corr_s[w][h][t] = the sum of token t's corrections
    // (fp32), and each block's QK^T accumulators of the hi columns start from
    // it (the lo columns start from the mean bias).  Lane L takes E consecutive entries, E =
    // ceil(n / 64): runs of one token inside a lane are summed in registers;
    // a run that closes inside the lane and is not its first belongs to the
    // lane alone (the list is sorted) and is written; the lane's first and
    // last runs may continue in the neighbouring lanes and are added with LDS
    // float atomics after the bias fill.  The first kPre entries of every
    // lane arrive in registers a segment ahead.
    constexpr int SB = kCT / 32;  // blocks per segment
    constexpr int kPre = 12;
    uint32_t gent[kPre];
#pragma unroll
    for (int k = 0; k < kPre; ++k) gent[k] = 0u;
    int gent_lo = 0, gent_n = 0;  // the segment whose entries gent holds: first entry, count
    float* const corr = &corr_s[w][0][0];
    // entries [lo, hi) of wave group j's side-list cover segment sg
    auto seg_range = [&](int j, int sg, int& lo, int& n) {
      lo = sg == 0 ? 0 : meta(j, 16 + sg * SB - 1);
      n = meta(j, 16 + min((sg + 1) * SB, nblk) - 1) - lo;
    };
    // the first kPre entries of every lane of [lo, lo + n) of the side-list
    // of group obase; a false `real` makes it a zero-size buffer (the loads
    // return zeros and touch no memory), so that every block load issues the
    // same loads and the waits on them stay exact
    auto load_entries = [&](int obase, int lo, int n, bool real) {
      const int E = (n + 63) >> 6;
      gent_lo = lo;
      gent_n = real ? n : 0;
      // the group's side-list as its own buffer: reads past its end return 0
      const __amdgpu_buffer_rsrc_t ro = buf_rsrc(oent_all + (size_t)(uint32_t)obase * cap,
                                                 real ? 4u * (uint32_t)cap : 0u);
      const int off = 4 * (lo + lane * E);
      const u32x4_t x0 = __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0);
      const u32x4_t x1 = __builtin_amdgcn_raw_buffer_load_b128(ro, off, 16, 0);
      const u32x4_t x2 = __builtin_amdgcn_raw_buffer_load_b128(ro, off, 32, 0);
      gent[0] = x0.x; gent[1] = x0.y; gent[2] = x0.z; gent[3] = x0.w;
      gent[4] = x1.x; gent[5] = x1.y; gent[6] = x1.z; gent[7] = x1.w;
      gent[8] = x2.x; gent[9] = x2.y; gent[10] = x2.z; gent[11] = x2.w;
    };
    auto load_seg_entries = [&](int j, int sg) {
      int lo, n;
      seg_range(j, sg, lo, n);
      load_entries(meta(j, 16 + TQK_NOB), lo, n, n > 0);
    };
    // with the loads of the block load_next fetches next (wave group jl,
    // block kbl): its segment's entries when it starts one
    auto load_block_entries = [&]() {
      const int sg = kbl / SB;
      const bool seg = kbl % SB == 0;
      const int lo = sg == 0 ? 0 : meta_l(16 + sg * SB - 1);
      const int n = meta_l(16 + min((sg + 1) * SB, nblk) - 1) - lo;
      load_entries(meta_l(16 + TQK_NOB), lo, n, seg && n > 0);
    };
    auto seg_pass = [&](int j, int sg) {
      // zero fill (tokens without outliers): lane L writes head hq
      // (= L mod GQ) for the tokens [NT (L / GQ), NT (L / GQ) + NT),
      // NT = kCT GQ / 64
      {
        constexpr int NT = kCT * GQ / 64;
        float4* row = reinterpret_cast<float4*>(corr + hq * kRow + NT * (lane / GQ));
#pragma unroll
        for (int i = 0; i < NT / 4; ++i) row[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      const int n = gent_n, lo = gent_lo;
      if (n == 0) return;
      const int E = (n + 63) >> 6;
      const int nl = n - lane * E;  // entries k < nl of this lane are in the list
      const __amdgpu_buffer_rsrc_t ro =
          buf_rsrc(oent_all + (size_t)(uint32_t)meta(j, 16 + TQK_NOB) * cap, 4u * (uint32_t)cap);
      const int t0 = kCT * sg;
      float acc[GQ], facc[GQ];
#pragma unroll
      for (int i = 0; i < GQ; ++i) acc[i] = facc[i] = 0.f;
      int tcur = -1, tfirst = -1;  // open run's token, first closed run's token (segment-relative)
      // One entry: a run closing inside the lane that is not its first is
      // stored at its token (an exec-masked store); the first is kept in facc.
      // An entry's LDS operands, the channel's group mean and q of every head
      // (fp16, exact), gathered for four entries before their arithmetic so
      // that the four gathers share one wait.  (Read for every lane: an
      // invalid entry's channel is still in range.)
      constexpr int kQW = (GQ + 1) / 2;
      struct EntryOps {
        float mean;
        uint32_t q[kQW];
      };
      auto gather = [&](uint32_t x, EntryOps& o) {
        const int jc = (int)(x & (uint32_t)(D - 1));
        o.mean = gsm_s[w][D + jc];
        if constexpr (GQ >= 4) {
#pragma unroll
          for (int i = 0; i < GQ; i += 4) {
            const uint2 q4 = *reinterpret_cast<const uint2*>(&qc_s[jc][i]);
            o.q[i / 2] = q4.x;
            o.q[i / 2 + 1] = q4.y;
          }
        } else if constexpr (GQ == 2) {
          o.q[0] = *reinterpret_cast<const uint32_t*>(&qc_s[jc][0]);
        } else {
          o.q[0] = qc_s[jc][0];
        }
      };
      auto entry = [&](int k, uint32_t x, const EntryOps& o) {
        // (an entry outside the segment's tokens is dropped, whatever the
        // list holds: every LDS index below stays in corr_s)
        const int tx = (int)((x >> 7) & 0xFFu) - t0;
        const bool valid = k < nl && (unsigned)tx < (unsigned)kCT;
        const int t = valid ? tx : -1;
        const bool close = t != tcur && tcur >= 0;
        const bool first = close && tfirst < 0;
        if (close && tfirst >= 0) {  // a run that closes inside the lane, not its first
#pragma unroll
          for (int i = 0; i < GQ; ++i) corr[i * kRow + tcur] = acc[i];
        }
#pragma unroll
        for (int i = 0; i < GQ; ++i) facc[i] = first ? acc[i] : facc[i];
        tfirst = first ? tcur : tfirst;
        const bool same = t == tcur;
        tcur = t;
        const float dv0 = (h2f((uint16_t)(x >> 16)) - o.mean) * qscale;
        const float dv = valid ? dv0 : 0.f;
        // q of every head at the entry's channel into fp32 FMAs
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          const _Float16 qv = __builtin_bit_cast(_Float16, (uint16_t)(o.q[i / 2] >> (16 * (i & 1))));
          acc[i] = fmaf((float)qv, dv, same ? acc[i] : 0.f);
        }
      };
      static_assert(kPre % 4 == 0, "entries in fours");
#pragma unroll
      for (int k0 = 0; k0 < kPre; k0 += 4) {
        if (k0 < E) {
          EntryOps o[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) gather(gent[k0 + u], o[u]);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (k0 + u < E) entry(k0 + u, gent[k0 + u], o[u]);
        }
      }
      for (int k = kPre; k < E; ++k) {  // long lists only; reads past the list return 0
        const uint32_t x = __builtin_amdgcn_raw_buffer_load_b32(ro, 4 * (lo + lane * E + k), 0, 0);
        EntryOps o;
        gather(x, o);
        entry(k, x, o);
      }
      // The lane's first and last runs may continue in its neighbours (the
      // list is sorted, so the lanes that share a token are consecutive, all
      // but the two ends holding that token only).  An inclusive scan of the
      // last-run sums over the lanes, segmented by the last-run token, gives
      // each lane the sum of its token's runs so far; the first run of a lane
      // takes its left neighbour's scan, and the last lane of a token's chain
      // stores it.  (LDS float atomics here serialise per lane.)
      float sv[GQ];
#pragma unroll
      for (int i = 0; i < GQ; ++i) sv[i] = acc[i];
      const int tl = tcur;                         // last run's token (-1: none)
      const int tf = tfirst >= 0 ? tfirst : tcur;  // first run's token
      // (every lane takes part in each shuffle: a lane outside the exec mask
      // has nothing to hand over; the edges are resolved after the shuffle)
      const int tl_up = __shfl_up(tl, 1), tf_dn = __shfl_down(tf, 1);
      const int tl_prev = lane > 0 ? tl_up : -1;
      // A lane's last run continues its left neighbour's only when every
      // entry of the lane is that one token: only such chains (a token over
      // three or more lanes) need the scan; otherwise each lane's sum is its own.
      if (__builtin_amdgcn_ballot_w64(tl >= 0 && tl == tl_prev) != 0) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const int kd = __shfl_up(tl, d);
          const bool add = lane >= d && kd == tl && tl >= 0;
#pragma unroll
          for (int i = 0; i < GQ; ++i) {
            const float v = __shfl_up(sv[i], d);
            sv[i] += add ? v : 0.f;
          }
        }
      }
      const int tf_next = lane < 63 ? tf_dn : -1;
      float sprev[GQ];
#pragma unroll
      for (int i = 0; i < GQ; ++i) sprev[i] = __shfl_up(sv[i], 1);
      if (tfirst >= 0) {
        // the first run ends inside this lane: complete with the carry-in
        const bool cin = tl_prev == tfirst;
#pragma unroll
        for (int i = 0; i < GQ; ++i) corr[i * kRow + tfirst] = facc[i] + (cin ? sprev[i] : 0.f);
      }
      if (tl >= 0 && tf_next != tl) {
#pragma unroll
        for (int i = 0; i < GQ; ++i) corr[i * kRow + tl] = sv[i];
      }
    };
    // QK^T accumulator start of block kb of the current group: hi columns
    // from corr_s (tokens 4lg..4lg+3 of tile A, then of tile B), lo columns
    // the group's mean bias
    const float* const init_base = is_hi ? corr + hq * kRow + 4 * lg : &bias_s[w][hq][0];
    const int init_step = is_hi ? 32 : 0;
    auto block_init = [&](int kb, floatx4_t& CA, floatx4_t& CB) {
      const float* p = init_base + init_step * (kb % SB);
      CA = *reinterpret_cast<const floatx4_t*>(p);
      CB = *reinterpret_cast<const floatx4_t*>(p + (is_hi ? 16 : 0));
    };

      // A operand of QK^T MFMA m from the lane's key bytes (a table row of a code
      // byte is {fp16 hi pair, fp16 lo pair} of its two channels)
      auto key_quad = [&](const uint4& k, int m) {
        uint32_t a0, a1;  // table addresses of channel pairs 2m, 2m + 1 of the chunk
        if constexpr (KB == 4) {
          // a code byte is the index: one v_perm puts it above the copy offset
          const uint32_t word = (m >> 1) == 0 ? k.x : (m >> 1) == 1 ? k.y : (m >> 1) == 2 ? k.z : k.w;
          const uint32_t q0 = 2u * (uint32_t)(m & 1);
          a0 = __builtin_amdgcn_perm(word, koff, 0x0C0C0000u | ((4u + q0) << 8));
          a1 = __builtin_amdgcn_perm(word, koff, 0x0C0C0000u | ((5u + q0) << 8));
        } else {
          uint32_t f0 = 0, f1 = 0;
          if constexpr (KB == 3) {
            switch (m) {
#define TQK_K3(M) case M: f0 = v3_field<2 * M>(k); f1 = v3_field<2 * M + 1>(k); break;
              TQK_K3(0) TQK_K3(1) TQK_K3(2) TQK_K3(3) TQK_K3(4) TQK_K3(5) TQK_K3(6) TQK_K3(7)
#undef TQK_K3
            }
          } else {
            // 4-bit fields 2m, 2m + 1 at bits 8m, 8m + 4 of the 64-bit chunk
            const uint32_t word = m < 4 ? k.x : k.y;
            f0 = (word >> (8 * (m & 3))) & 15u;
            f1 = (word >> (8 * (m & 3) + 4)) & 15u;
          }
          a0 = (f0 << 8) | koff;
          a1 = (f1 << 8) | koff;
        }
        const uint2 t0 = *reinterpret_cast<const uint2*>(klut + a0);
        const uint2 t1 = *reinterpret_cast<const uint2*>(klut + a1);
        H8 r;
        r.u[0] = t0.x;
        r.u[1] = t0.y;
        r.u[2] = t1.x;
        r.u[3] = t1.y;
        return r;
      };

      // B operand of PV MFMA nt: single fp16 centroids of tokens 0..3 of the
      // lane's value unit in tile A (channel 8n + nt), then of tile B:
      // k-slots [A t0 t1 t2 t3, B t0 t1 t2 t3], matching the weight operand.
      auto val_op = [&](const uint4& uA, const uint4& uB, auto ntc) {
        constexpr int nt = decltype(ntc)::value;
        H8 r;
        if constexpr (LutGeom<KB, VB, GQ>::kPair6) {
          // 6-bit fields 2nt (tokens 0, 1) and 2nt + 1 (tokens 2, 3)
          auto lk = [&](uint32_t f) { return *reinterpret_cast<const uint32_t*>(lut + ((f << 8) | voff)); };
          r.u[0] = lk(v3_field<2 * nt>(uA));
          r.u[1] = lk(v3_field<2 * nt + 1>(uA));
          r.u[2] = lk(v3_field<2 * nt>(uB));
          r.u[3] = lk(v3_field<2 * nt + 1>(uB));
        } else if constexpr (VB == 3) {
          // the 12-bit field nt (bits 12nt..12nt+11 of the 96-bit unit) is its
          // own table index: the address is the field times 8, taken with one
          // funnel shift that leaves it at bit 3 and one mask (the table sits
          // at LDS offset 0)
          constexpr int o = 12 * nt, w = o / 32, sh = o % 32;
          auto addr = [&](const uint4& u) -> uint32_t {
            if constexpr (sh == 0) {
              return (u4_word<w>(u) << 3) & 0x7FF8u;
            } else if constexpr (sh + 12 <= 32) {
              return (u4_word<w>(u) >> (sh - 3)) & 0x7FF8u;
            } else {
              return __builtin_amdgcn_alignbit(u4_word<w + 1>(u), u4_word<w>(u), sh - 3) & 0x7FF8u;
            }
          };
          const uint2 x = *reinterpret_cast<const uint2*>(lut + addr(uA));
          const uint2 y = *reinterpret_cast<const uint2*>(lut + addr(uB));
          r.u[0] = x.x;
          r.u[1] = x.y;
          r.u[2] = y.x;
          r.u[3] = y.y;
        } else if constexpr (VB == 2) {
          // code byte nt (four 2-bit codes) of the 8-byte unit
          const uint32_t sel = 0x0C0C0000u | ((4u + (uint32_t)(nt & 3)) << 8);
          const uint32_t ax = __builtin_amdgcn_perm(nt < 4 ? uA.x : uA.y, voff, sel);
          const uint32_t ay = __builtin_amdgcn_perm(nt < 4 ? uB.x : uB.y, voff, sel);
          const uint2 x = *reinterpret_cast<const uint2*>(lut + ax);
          const uint2 y = *reinterpret_cast<const uint2*>(lut + ay);
          r.u[0] = x.x;
          r.u[1] = x.y;
          r.u[2] = y.x;
          r.u[3] = y.y;
        } else {
          // code bytes 2nt (tokens 0, 1) and 2nt + 1 (tokens 2, 3) of the 16-byte unit
          const uint32_t s0 = 0x0C0C0000u | ((4u + 2u * (uint32_t)(nt & 1)) << 8);
          const uint32_t s1 = 0x0C0C0000u | ((5u + 2u * (uint32_t)(nt & 1)) << 8);
          const uint32_t wa = u4_word<nt / 2>(uA), wb = u4_word<nt / 2>(uB);
          r.u[0] = *reinterpret_cast<const uint32_t*>(lut + __builtin_amdgcn_perm(wa, voff, s0));
          r.u[1] = *reinterpret_cast<const uint32_t*>(lut + __builtin_amdgcn_perm(wa, voff, s1));
          r.u[2] = *reinterpret_cast<const uint32_t*>(lut + __builtin_amdgcn_perm(wb, voff, s0));
          r.u[3] = *reinterpret_cast<const uint32_t*>(lut + __builtin_amdgcn_perm(wb, voff, s1));
        }
        return r;
      };

      // Software pipeline over a wave's blocks.  Step i starts with the QK^T
      // accumulators of block i (computed in step i - 1 from the initial
      // values of its group's corr_s): it runs block i's softmax, and
      // interleaves block i's PV with block i + 1's QK^T so that the table
      // reads of one overlap the MFMAs of the other.  When block i + 1 starts
      // a group, its weights and corr_s are built in between.
      floatx4_t CAn, CBn;       // QK^T of the block computed next
      auto key_tile = [&](const uint4& k, H8 (&x)[8]) {
#pragma unroll
        for (int m = 0; m < 8; ++m) x[m] = key_quad(k, m);
      };
      auto qk_tile = [&](const H8 (&x)[8], floatx4_t& C) {
#pragma unroll
        for (int m = 0; m < 8; ++m) C = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[m].h, Bw[m].h, C, 0, 0, 0);
      };
      auto val_block = [&](const uint4& uA, const uint4& uB, H8 (&v)[8]) {
        v[0] = val_op(uA, uB, IntC<0>{});
        v[1] = val_op(uA, uB, IntC<1>{});
        v[2] = val_op(uA, uB, IntC<2>{});
        v[3] = val_op(uA, uB, IntC<3>{});
        v[4] = val_op(uA, uB, IntC<4>{});
        v[5] = val_op(uA, uB, IntC<5>{});
        v[6] = val_op(uA, uB, IntC<6>{});
        v[7] = val_op(uA, uB, IntC<7>{});
      };
      // PV over the whole 32-token block: k = the lane group's 8 tokens
      auto pv_block = [&](const H8& pw, const H8 (&v)[8]) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) st.O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pw.h, v[nt].h, st.O[nt], 0, 0, 0);
      };
      // blk1: block index of block i + 1 inside its group (whose weights and
      // corrections are built before the step when it starts a segment)
      auto process = [&](const ColdBlock<VB>& cur, const ColdBlock<VB>& nx1, int blk1) {
        const floatx4_t CA = CAn, CB = CBn;
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[i] = pair_sum(CA[i]);
          sc[4 + i] = pair_sum(CB[i]);
        }
        if constexpr (PK) {
          // score = |k| * (q_rot . centroids)
          sc[0] *= row_bcast<0>(cur.kn);
          sc[1] *= row_bcast<1>(cur.kn);
          sc[2] *= row_bcast<2>(cur.kn);
          sc[3] *= row_bcast<3>(cur.kn);
          sc[4] *= row_bcast<4>(cur.kn);
          sc[5] *= row_bcast<5>(cur.kn);
          sc[6] *= row_bcast<6>(cur.kn);
          sc[7] *= row_bcast<7>(cur.kn);
        }
        float p[8];
        softmax_block<GQ>(st, sc, p, lg);
        // A operand of PV: weight times value norm of the lane's 8 tokens
        // (tile A 4lg..4lg+3, tile B 4lg..4lg+3) for head hq, fp16 hi in rows
        // c < 8, the fp16 residual in rows c >= 8
        const H8 pw = split8(p[0] * row_bcast<0>(cur.nv), p[1] * row_bcast<1>(cur.nv),
                             p[2] * row_bcast<2>(cur.nv), p[3] * row_bcast<3>(cur.nv),
                             p[4] * row_bcast<4>(cur.nv), p[5] * row_bcast<5>(cur.nv),
                             p[6] * row_bcast<6>(cur.nv), p[7] * row_bcast<7>(cur.nv), lo_sel);
        H8 vv[8], xa[8], xb[8];
        // (no scheduling fences between the phases: the compiler's own
        // interleaving measured faster and needs fewer registers)
        val_block(cur.uA, cur.uB, vv);
        key_tile(nx1.kA, xa);
        pv_block(pw, vv);
        block_init(blk1, CAn, CBn);
        qk_tile(xa, CAn);
        key_tile(nx1.kB, xb);
        qk_tile(xb, CBn);
      };

    // A ring of kColdBuf buffers, kColdBuf - 1 blocks in flight: step i
    // issues the loads of block i + kColdBuf - 1 and computes block i.
    int jp = 0, kbp = kb0;  // computed block: wave group jp, block kbp
    int si = 0;             // stream index of the computed block
    // Waves w and w + 4 share a SIMD, and its arbiter favours the older wave
    // when both can issue: with whole-group shares, waves 4-7 finished ~15 us
    // after waves 0-3 at the headline and the SIMDs ended with one wave each.
    // Waves 4-7 raise their issue priority for three blocks of every four
    // (half of them left the older waves ~7 us ahead; all of them turned the
    // order round), which evens the pairs out (issue order only: the results
    // are the same).
    const bool pair_prio = wu >= 4 && a.wave_blocks == 0;
    auto step = [&](const ColdBlock<VB>& cur, ColdBlock<VB>& nxt, const ColdBlock<VB>& nx1) {
      store_group_stats();  // block i + 1's group
      const bool starts = kbp + 1 == nblk;  // block i + 1 starts wave group jp + 1
      const int kb1 = starts ? 0 : kbp + 1, j1 = starts ? jp + 1 : jp;
      // (after the wave's last block there is no block i + 1: nothing to
      // build, and process's QK^T of it runs on a stale buffer, unused)
      if (__builtin_expect(si + 1 < T && kb1 % SB == 0, 0)) {
        // block i + 1 starts a segment (and maybe its group): weights and
        // bias, then the segment's corrections from the entries loaded with
        // the block in the previous step
        wave_sync();
        if (starts) begin_group();
        seg_pass(j1, kb1 / SB);
      }
      load_group_stats(meta_l(16 + TQK_NOB));  // group of the block load_next fetches now
      wave_sync();
      load_block_entries();
      load_next(nxt);
      process(cur, nx1, kb1);
      if (++kbp == nblk) {
        kbp = 0;
        ++jp;
      }
      ++si;
      // waves 4-7: issue priority up for three blocks of every four
      if (pair_prio) {
        if ((si & 3) == 3)
          __builtin_amdgcn_s_setprio(0);
        else if ((si & 3) == 0)
          __builtin_amdgcn_s_setprio(1);
      }
    };
    // The first group: stats and the side-list of the first block's segment
    // synchronously; the group of the second block's stats into the pending
    // registers; the first block's codes are requested with them, so that
    // they arrive while its group's weights and corrections are built (the
    // side-list entries of its segment are the ones just loaded).  A wave
    // that reads its own metadata rows issues these loads before the
    // set-up's workgroup barrier, which then waits for LDS only.
    ColdBlock<VB> ring[kColdBuf];
    auto first_loads = [&]() {
      load_group_stats(meta(0, 16 + TQK_NOB));
      load_seg_entries(0, kb0 / SB);
      load_next(ring[0]);
    };
    // (one load site, so that the waits on these loads stay exact; own_rows
    // is the same for every wave, so each wave takes one barrier)
    if (!own_rows) {
      lds_barrier();
      load_meta(0);
    }
    if (T > 0) first_loads();
    if (own_rows) lds_barrier();
    if (T > 0) {
      const int j1 = (kb0 + min(1, T - 1)) / nblk;
      const int sg0 = kb0 / SB;
      store_group_stats();
      wave_sync();
      begin_group();
      seg_pass(0, sg0);
      load_group_stats(meta(j1, 16 + TQK_NOB));
#pragma unroll
      for (int s = 1; s < kColdBuf - 1; ++s) {
        load_block_entries();
        load_next(ring[s]);
      }
      wave_sync();
      {
        H8 x[8];
        block_init(kb0, CAn, CBn);
        key_tile(ring[0].kA, x);
        qk_tile(x, CAn);
        key_tile(ring[0].kB, x);
        qk_tile(x, CBn);
      }
      if (pair_prio) __builtin_amdgcn_s_setprio(1);
      for (int i = 0; i < T; i += kColdBuf) {
#pragma unroll
        for (int s = 0; s < kColdBuf; ++s) {
          if (i + s >= T) break;
          step(ring[s], ring[(s + kColdBuf - 1) % kColdBuf], ring[(s + 1) % kColdBuf]);
        }
      }
    }
  }
  // ---- this split's share of the fp16 hot window: tokens [n_cold, L) from
  // the ring in 32-token blocks, block split * 8 + w onwards, in a fresh state
  // (its partial is not rotated back, unlike the coded one).  The coded state
  // waits in registers meanwhile: the code table, where the waves' states are
  // folded, is still read by waves that have not finished their groups.
  __builtin_amdgcn_s_setprio(0);
  const WaveState cst = st;
  reset_state(st);
  {
    const int n_cold = ng * G, R = d.hot_ring;
    const size_t hbase = ((size_t)b * Hkv + h) * R;
    const int nhb = (L - n_cold + 31) / 32;
    // B operand of QK^T: q (fp16, exact) of head c for channels 32ks + 8lg + e
    H8 Bq[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      Bq[ks].v = *reinterpret_cast<const uint4*>(&qf_s[hq][32 * ks + 8 * lg]);
    for (int hb = split * kMWaves + w; hb < nhb; hb += a.n_cold_splits * kMWaves) {
      // n_cold and the ring size are multiples of 32: the block's 32 ring rows
      // are consecutive and inside the ring, so every row is loaded (keys and
      // values together) and rows at or past L are masked afterwards
      const int t0 = n_cold + 32 * hb;
      const uint16_t* kr = static_cast<const uint16_t*>(a.p.hot_k) + (hbase + (t0 % R)) * D;
      const uint16_t* vr = static_cast<const uint16_t*>(a.p.hot_v) + (hbase + (t0 % R)) * D;
      H8 ka[4], kb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        ka[ks].v = *reinterpret_cast<const uint4*>(kr + (size_t)c * D + 32 * ks + 8 * lg);
        kb[ks].v = *reinterpret_cast<const uint4*>(kr + (size_t)(16 + c) * D + 32 * ks + 8 * lg);
      }
      // values: token e of this lane (tile A 4lg+e, tile B 16+4lg+e), channels 8c..8c+7
      uint4 vv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tt = (e < 4) ? 4 * lg + e : 16 + 4 * lg + (e - 4);
        vv[e] = *reinterpret_cast<const uint4*>(vr + (size_t)tt * D + 8 * c);
      }
      floatx4_t CA = {0.f, 0.f, 0.f, 0.f}, CB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        CA = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks].h, Bq[ks].h, CA, 0, 0, 0);
        CB = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[ks].h, Bq[ks].h, CB, 0, 0, 0);
      }
      float s[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = (t0 + 4 * lg + i < L) ? CA[i] * qscale : -INFINITY;
        s[4 + i] = (t0 + 16 + 4 * lg + i < L) ? CB[i] * qscale : -INFINITY;
      }
      float p[8];
      softmax_block<GQ>(st, s, p, lg);
      H8 pa;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 hi = (_Float16)p[e];
        pa.h[e] = is_hi ? hi : (_Float16)(p[e] - (float)hi);
      }
      // rows past L: zero (whatever the ring holds there, 0 * inf would be NaN)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tt = (e < 4) ? 4 * lg + e : 16 + 4 * lg + (e - 4);
        if (t0 + tt >= L) vv[e] = make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        H8 vb;
        const uint32_t sel = (nt & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&vv[2 * k]);
          const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&vv[2 * k + 1]);
          vb.u[k] = __builtin_amdgcn_perm(v1[nt >> 1], v0[nt >> 1], sel);
        }
        st.O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa.h, vb.h, st.O[nt], 0, 0, 0);
      }
    }
  }

  // ---- the two partials.  A wave's state goes to (m_w[head], l_w[head],
  // co_w[head][D]); accumulator rows r < 8 hold the fp16-hi weights of head r,
  // rows r >= 8 the lo weights of head r - 8, summed onto the same row.
  auto put_state = [&](const WaveState& x, float* m_w, float* l_w, float* co_w) {
    const float lsum = colgroup_sum(x.l);
    if (lg == 0 && c < GQ) {
      m_w[c] = x.m;
      l_w[c] = lsum;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * lg + i;
      if (r < GQ) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) co_w[r * D + 8 * c + nt] = x.O[nt][i];
      }
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * lg + i;
      if (r >= 8 && r < 8 + GQ) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) co_w[(r - 8) * D + 8 * c + nt] += x.O[nt][i];
      }
    }
  };
  // hot state: this wave's own stats slot and corrections (no longer read)
  float* const hm = &gsm_s[0][0];                 // wave ww: hm[ww * 2D + i]
  float* const hco = &corr_s[0][0][0];            // wave ww: hco[ww * GQ * kRow + i * D + j]
  constexpr int kHmStride = 2 * D, kHcoStride = GQ * kRow;
  static_assert(kCT >= D, "hot-state area");
  put_state(st, hm + w * kHmStride, hm + w * kHmStride + D, hco + w * kHcoStride);
  // coded state: the code table's area, once every wave is past its groups
  __syncthreads();
  float* const cm = reinterpret_cast<float*>(lut);  // [8][GQ]
  float* const cl = cm + kMWaves * GQ;              // [8][GQ]
  float* const co = cl + kMWaves * GQ;              // [8][GQ][D]
  put_state(cst, cm + w * GQ, cl + w * GQ, co + w * GQ * D);
  __syncthreads();
  // fold the eight waves of each: partial n_cold_splits * hot + split.
  // With one coded split per (seq, kv head) and 4 or 8 heads, the thread
  // that folds (coded/hot, head i, channel j) is the one that merges head i
  // for channel j below (u = tid / D): the two partials stay in its
  // registers (dvm/dvl/dva, the values the stores would write) and the
  // merge reads them there -- no stores, arrival or reloads.
  const int ns = a.n_cold_splits + a.n_hot_splits;
  constexpr int kFoldIt = (2 * GQ * D + kMThreads - 1) / kMThreads;
  const bool direct = (GQ == 4 || GQ == 8) && a.out != nullptr && a.n_cold_splits == 1;
  float dvm[kFoldIt], dvl[kFoldIt], dva[kFoldIt];
#pragma unroll
  for (int it = 0; it < kFoldIt; ++it) {
    dvm[it] = -INFINITY;
    dvl[it] = 0.f;
    dva[it] = 0.f;
    const int x = tid + it * kMThreads;
    if (x >= 2 * GQ * D) continue;
    const int hot = x >= GQ * D;
    const int i = (x % (GQ * D)) / D, j = x % D;
    if (i >= gq) continue;
    const float* mp = hot ? hm + i : cm + i;
    const float* lp = hot ? hm + D + i : cl + i;
    const float* op = hot ? hco + i * D + j : co + i * D + j;
    const int ms = hot ? kHmStride : GQ, os = hot ? kHcoStride : GQ * D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kMWaves; ++ww)
      if (lp[ww * ms] > 0.f) M = fmaxf(M, mp[ww * ms]);
    float den = 0.f, acc = 0.f;
    if (M > -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < kMWaves; ++ww) {
        const float l = lp[ww * ms];
        if (l > 0.f) {
          const float wt = __builtin_amdgcn_exp2f(mp[ww * ms] - M);
          den += l * wt;
          acc += op[ww * os] * wt;
        }
      }
    }
    dvm[it] = M * 0.6931471805599453f;  // back to the natural-log domain of the partials
    dvl[it] = den;
    dva[it] = acc;
    if (!direct) {
      const size_t o = ((size_t)b * Hq + h * gq + i) * ns + (hot ? a.n_cold_splits : 0) + split;
      st_agent(a.pacc + o * D + j, acc);
      if (j == 0) {
        st_agent(a.pm + o, dvm[it]);
        st_agent(a.pl + o, den);
      }
    }
  }

  if (a.out == nullptr) return;

  // ---- in-kernel merge: the last of the (seq, kv head)'s n_cold_splits
  // workgroups to finish combines their partials (same arithmetic as
  // tqk_merge).  The partials were stored with agent-scope coherent stores
  // and are read with agent-scope coherent loads (the workgroups may sit on
  // different XCDs, each with its own L2; device-scope fences would write
  // back and invalidate whole L2s instead, measured slower).  Every thread
  // waits for its stores to complete before the arrival is counted, and the
  // last arrival's loads are issued after it has read the count.  The counter
  // wraps back to zero on the last arrival, so it is zero for the next call.
  __shared__ int last_s;
  if (!direct) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are done
    __syncthreads();
    // acquire-release at agent scope: the workgroup's partial stores (ordered
    // before this RMW by the barrier above) are released to the last arrival,
    // whose loads below are ordered after its acquire
    if (tid == 0)
      last_s = __builtin_amdgcn_atomic_inc32(a.arrive + (size_t)b * Hkv + h,
                                             (uint32_t)(a.n_cold_splits - 1), __ATOMIC_ACQ_REL,
                                             "agent") == (uint32_t)(a.n_cold_splits - 1);
    __syncthreads();
    if (!last_s) return;
  } else {
    __syncthreads();  // every wave past the fold's reads of the code table's area (Pi goes there)
  }
  {
    // thread (u, j): query heads u, u + 4 for channel j; the coded sums go to
    // q_h_s.  Up to kMergeFast splits, every partial load is issued before
    // the first is used (each is a round trip to memory).
    const int j = tid % D, u = tid / D;
    constexpr int NH = (GQ + 3) / 4;
    float hr[NH], den[NH];
    auto combine = [&](int r, int qi, const float (&vl)[kMergeFast], const float (&vm)[kMergeFast],
                       const float (&va)[kMergeFast]) {
      float M = -INFINITY;
#pragma unroll
      for (int s = 0; s < kMergeFast; ++s)
        if (vl[s] > 0.f) M = fmaxf(M, vm[s]);
      float dn = 0.f, cr = 0.f, hh = 0.f;
#pragma unroll
      for (int s = 0; s < kMergeFast; ++s) {
        if (vl[s] > 0.f) {
          const float wt = __expf(vm[s] - M);
          dn += vl[s] * wt;
          const float x = va[s] * wt;
          if (s < a.n_cold_splits) cr += x; else hh += x;
        }
      }
      q_h_s[qi][j] = cr;
      hr[r] = hh;
      den[r] = dn;
    };
#pragma unroll
    for (int r = 0; r < NH; ++r) hr[r] = den[r] = 0.f;
    const bool fast = ns <= kMergeFast;
    // hot partials past the hot window's blocks (split s takes blocks 8s + w
    // onwards) are empty
    const int hot_live = min(a.n_cold_splits, ((L - ng * G + 31) / 32 + kMWaves - 1) / kMWaves);
    float vl[NH][kMergeFast], vm[NH][kMergeFast], va[NH][kMergeFast];
    if (direct) {
      // split 0 = the coded partial (fold iteration r), split 1 = the hot one
      // (iteration kFoldIt / 2 + r), as the stores would have laid them out
#pragma unroll
      for (int r = 0; r < NH; ++r) {
#pragma unroll
        for (int s2 = 0; s2 < kMergeFast; ++s2) {
          const int itc = s2 == 0 ? r : kFoldIt / 2 + r;
          vl[r][s2] = s2 < 2 ? dvl[itc < kFoldIt ? itc : 0] : 0.f;
          vm[r][s2] = s2 < 2 ? dvm[itc < kFoldIt ? itc : 0] : -INFINITY;
          va[r][s2] = s2 < 2 ? dva[itc < kFoldIt ? itc : 0] : 0.f;
        }
      }
    } else if (fast) {
#pragma unroll
      for (int r = 0; r < NH; ++r) {
        const int qi = u + 4 * r;
        const size_t base = ((size_t)b * Hq + h * gq + qi) * ns;
#pragma unroll
        for (int s = 0; s < kMergeFast; ++s) {
          const bool ok = qi < gq && s < ns;
          vl[r][s] = ok ? ld_agent(a.pl + base + s) : 0.f;
          vm[r][s] = ok ? ld_agent(a.pm + base + s) : -INFINITY;
          va[r][s] = ok ? ld_agent(a.pacc + (base + s) * D + j) : 0.f;
        }
      }
    }
    {
      // Pi (64 KiB) into the code table's area, its wide loads issued behind
      // the partial loads and before any store
      constexpr int NV = D * D / 4 / kMThreads;
      float4 v[NV];
#pragma unroll
      for (int r = 0; r < NV; ++r) v[r] = reinterpret_cast<const float4*>(a.p.pi)[tid + r * kMThreads];
#pragma unroll
      for (int r = 0; r < NV; ++r) reinterpret_cast<float4*>(lut)[tid + r * kMThreads] = v[r];
    }
    const float* const pi_s = reinterpret_cast<const float*>(lut);
    if (fast) {
#pragma unroll
      for (int r = 0; r < NH; ++r)
        if (u + 4 * r < gq) combine(r, u + 4 * r, vl[r], vm[r], va[r]);
    } else {
#pragma unroll
      for (int r = 0; r < NH; ++r) {
        const int qi = u + 4 * r;
        if (qi < gq) {
          const size_t base = ((size_t)b * Hq + h * gq + qi) * ns;
          float M, dn, cr, hh;
          merge_chunked<D>([](const float* p) { return ld_agent(p); }, a.pl, a.pm, a.pacc, base, ns,
                           a.n_cold_splits + hot_live, a.n_cold_splits, j, M, dn, cr, hh);
          q_h_s[qi][j] = cr;
          hr[r] = hh;
          den[r] = dn;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NH; ++r) {
      const int qi = u + 4 * r;
      if (qi < gq) {
        float o = hr[r];
#pragma unroll 8
        for (int k = 0; k < D; ++k) o += q_h_s[qi][k] * pi_s[k * D + j];
        a.out[((size_t)b * Hq + h * gq + qi) * D + j] = o / den[r];
      }
    }
  }
}

// One workgroup per (kv head, sequence): thread (half, j) merges the splits of
// query heads half, half + 2, ... for channel j, rotates their coded part back
// (sum_k acc[k] * Pi[k][j]) and adds the hot part (turboquant_pro/kv_fused.py:139-153).
// Pi is staged in LDS once (every thread's wide loads issued before its
// stores) and shared by the GQ query heads; at head_dim 256 (256 KiB of Pi)
// the rotation reads Pi from global memory instead.
template <int D>
__global__ __launch_bounds__(2 * D) void tqk_merge(MergeArgs a) {
  constexpr int kMergeThreads = 2 * D;
  constexpr bool kPiLds = D <= 128;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int j = tid & (D - 1), half = tid / D;
  const int GQ = a.n_q_heads / a.n_kv_heads;
  __shared__ __align__(16) float pi_s[kPiLds ? D * D : 4];
  __shared__ float crot_s[8][D];
  // every partial load of the thread's heads in flight at once when the
  // split count allows (the partials were just written: each round trip is an
  // L2 latency), then Pi's wide loads, then the combine
  const bool fast = a.n_splits <= kMergeFast;
  float vl[4][kMergeFast], vm[4][kMergeFast], va[4][kMergeFast];
  if (fast) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qi = half + 2 * u;
      const size_t base = ((size_t)b * a.n_q_heads + h * GQ + qi) * a.n_splits;
#pragma unroll
      for (int s = 0; s < kMergeFast; ++s) {
        const bool ok = qi < GQ && s < a.n_splits;
        vl[u][s] = ok ? a.pl[base + s] : 0.f;
        vm[u][s] = ok ? a.pm[base + s] : -INFINITY;
        va[u][s] = ok ? a.pacc[(base + s) * D + j] : 0.f;
      }
    }
  }
  if constexpr (kPiLds) {
    constexpr int NV = D * D / 4 / kMergeThreads;
    float4 v[NV];
#pragma unroll
    for (int r = 0; r < NV; ++r) v[r] = reinterpret_cast<const float4*>(a.pi)[tid + r * kMergeThreads];
#pragma unroll
    for (int r = 0; r < NV; ++r) reinterpret_cast<float4*>(pi_s)[tid + r * kMergeThreads] = v[r];
  }
  const float* __restrict__ pim = kPiLds ? pi_s : a.pi;
  float hr[4], den[4], mx[4];
  // merge of query head qi's splits for channel j: M = max m over splits with
  // l > 0, weights e^{m - M}; cold accumulators summed apart from the hot one
  auto combine = [&](int u, int qi, const float* vl, const float* vm, const float* va, int ns) {
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s)
      if (vl[s] > 0.f) M = fmaxf(M, vm[s]);
    float dn = 0.f, cr = 0.f, hh = 0.f;
    for (int s = 0; s < ns; ++s) {
      if (vl[s] > 0.f) {
        const float wt = __expf(vm[s] - M);
        dn += vl[s] * wt;
        const float v = va[s] * wt;
        if (s < a.n_cold_splits) cr += v; else hh += v;
      }
    }
    crot_s[qi][j] = cr;
    hr[u] = hh;
    den[u] = dn;
    mx[u] = M;
  };
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    hr[u] = den[u] = 0.f;
    mx[u] = -INFINITY;
  }
  if (fast) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qi = half + 2 * u;
      if (qi < GQ) combine(u, qi, vl[u], vm[u], va[u], kMergeFast);
    }
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qi = half + 2 * u;
      if (qi < GQ) {
        const size_t base = ((size_t)b * a.n_q_heads + h * GQ + qi) * a.n_splits;
        float M, dn, cr, hh;
        merge_chunked<D>([](const float* p) { return *p; }, a.pl, a.pm, a.pacc, base, a.n_splits,
                         a.n_splits, a.n_cold_splits, j, M, dn, cr, hh);
        crot_s[qi][j] = cr;
        hr[u] = hh;
        den[u] = dn;
        mx[u] = M;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int qi = half + 2 * u;
    if (qi < GQ) {
      float o = hr[u];
      // (Pi from global memory at head_dim 256: 32 rows' loads in flight per
      // batch; same sum, in row order)
      constexpr int kRotU = kPiLds ? 8 : 32;
#pragma unroll kRotU
      for (int k = 0; k < D; ++k) o += crot_s[qi][k] * pim[k * D + j];
      const size_t qh = (size_t)b * a.n_q_heads + h * GQ + qi;
      if (a.out) {
        a.out[qh * D + j] = o / den[u];
      } else {
        a.acc_out[qh * D + j] = o;
        if (j == 0) {
          a.m_out[qh] = mx[u];
          a.l_out[qh] = den[u];
        }
      }
    }
  }
}

// The MFMA kernel needs tiled value codes and a hot ring of whole 32-token blocks.
// (its loads use 32-bit buffer offsets: one head's page region stays below 4 GiB)
__host__ __device__ inline bool mfma_path(const tqk_cache_desc& d) {
  return v_tiled(d.group_tokens, d.page_tokens, d.head_dim, d.input_f32) && (d.hot_ring % 32 == 0) &&
         (long long)d.n_pages * d.page_tokens * (TQK_D / 2) < (1LL << 32);
}

// Sequences the arrival counters of a workspace cover: the page pool's page
// count (a pool of whole sequences holds at least one page per sequence).  A
// decode call may take at most this many sequences.
inline int counter_seqs(const tqk_cache_desc& d) { return d.n_pages; }

struct Plan {
  int n_cold_splits, n_hot_splits, groups_per_split, hot_per_split;
  int wave_blocks;  // MFMA kernel: blocks per wave of a split smaller than 8 groups, else 0
  size_t counter_bytes;  // arrival counters at the workspace's start, then the partials
  size_t partial_bytes;  // the split partials (m, l, acc)
  size_t ws_bytes;
};

// Where one call's arrival counters and split partials live: the caller's
// workspace, or the library's scratch array for tqk_decode_noalloc.
struct WsView {
  uint32_t* arrive;
  void* partials;
};

// compute units of the current device (the plan sizes the launch for them),
// queried once per device and process
constexpr int kMaxDevices = 64;
int device_cus() {
  static std::atomic<int> cus[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
    n = 256;
  cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

Plan make_plan(const tqk_cache_desc* d, int batch, int max_len) {
  Plan pl{};
  const int G = d->group_tokens;
  const int ngmax = n_groups_of(max_len, d->hot_window, G);
  const int hot_max = max_len < d->hot_window ? max_len : d->hot_window;
  pl.hot_per_split = kThreads;
  pl.n_hot_splits = (hot_max + kThreads - 1) / kThreads;
  if (pl.n_hot_splits < 1) pl.n_hot_splits = 1;
  const long units = (long)batch * d->n_kv_heads * (ngmax > 0 ? ngmax : 0);
  int gps;
  if (mfma_path(*d)) {
    // MFMA kernel: one workgroup per CU at a time (its LDS), eight waves
    // each walking every eighth group of the split.  Pick the groups per wave
    // (<= kMaxGPS / 8: a split's group metadata lives in LDS) that minimises
    // rounds of CUs x groups per wave in the longest split, plus about a
    // third of a group of per-workgroup set-up (code tables, fold).
    const int ncu = device_cus();
    double best = 1e30;
    int gpw_best = 1;
    for (int gpw = 1; gpw <= kMaxGPS / kMWaves; ++gpw) {
      const long g = (long)kMWaves * gpw;
      const long items = (long)batch * d->n_kv_heads * ((ngmax + g - 1) / g);
      const long rounds = (items + ncu - 1) / ncu;
      const long per_wave = ((ngmax < g ? ngmax : g) + kMWaves - 1) / kMWaves;
      const double cost = (double)rounds * ((double)per_wave + 0.35);
      if (cost < best - 1e-9) {
        best = cost;
        gpw_best = gpw;
      }
    }
    gps = kMWaves * gpw_best;
    // Short contexts: splits of 1, 2 or 4 groups whose blocks the eight waves
    // share (wave_blocks each) put more workgroups on the CUs when there are
    // few (seq, kv head) pairs (same cost model, in groups per wave)
    const int nblk = d->group_tokens / 32;
    for (int g = 1; g < kMWaves; g *= 2) {
      if ((g * nblk) % kMWaves) continue;
      const long items = (long)batch * d->n_kv_heads * ((ngmax + g - 1) / g);
      const long rounds = (items + ncu - 1) / ncu;
      const double cost = (double)rounds * ((double)g / kMWaves + 0.35);
      if (cost < best - 1e-9) {
        best = cost;
        gps = g;
        pl.wave_blocks = g * nblk / kMWaves;
      }
    }
  } else {
    // VALU kernel: a workgroup pays its set-up (query, code tables, the
    // split's partial, the merge's share) once for its gps groups, about a
    // group's time, and about three of its workgroups fit a CU.  Pick gps from
    // the bound of at most 4096 coded workgroups (which bounds the partials)
    // up to 8x that, minimising rounds of the CUs times (gps + 1), the hot
    // splits' workgroups counted in the rounds.
    const long slots = 3L * device_cus();
    const long pairs = (long)batch * d->n_kv_heads;
    const int g_lo = units > 4096 ? (int)((units + 4095) / 4096) : 1;
    const int g_hi = ngmax > g_lo ? (8 * g_lo < ngmax ? 8 * g_lo : ngmax) : g_lo;
    double best = 1e30;
    gps = g_lo;
    for (int g = g_lo; g <= g_hi; ++g) {
      const long blocks = pairs * ((ngmax + g - 1) / g + pl.n_hot_splits);
      const long rounds = (blocks + slots - 1) / slots;
      const double cost = (double)rounds * (g + 1);
      if (cost < best - 1e-9) {
        best = cost;
        gps = g;
      }
    }
  }
  pl.groups_per_split = gps;
  pl.n_cold_splits = ngmax > 0 ? (ngmax + gps - 1) / gps : 0;
  if (mfma_path(*d)) {
    // every MFMA workgroup also takes a share of the hot window and writes a
    // hot partial of its own: one split at least, as many hot partials
    if (pl.n_cold_splits < 1) pl.n_cold_splits = 1;
    pl.n_hot_splits = pl.n_cold_splits;
  }
  const size_t ns = (size_t)(pl.n_cold_splits + pl.n_hot_splits);
  const size_t per = (size_t)batch * d->n_q_heads * ns;
  // One counter per (seq, kv head) for counter_seqs() sequences, a bound that
  // depends on the descriptor only: the counter region never moves or grows
  // between calls, so no plan's partials ever land on a counter and the
  // counters stay zero between calls whatever the batch and split counts.
  const size_t n_counters = (size_t)counter_seqs(*d) * d->n_kv_heads;
  pl.counter_bytes = (n_counters * sizeof(uint32_t) + 255) & ~(size_t)255;
  pl.partial_bytes = per * sizeof(float) * (2 + d->head_dim);
  pl.ws_bytes = pl.counter_bytes + pl.partial_bytes + 256;
  return pl;
}

template <int GQ, int KB>
void launch_mfma_kb(const DecodeArgs& a, dim3 g1, hipStream_t st) {
  if (a.d.key_grid == 2)  // PolarQuant keys: value_bits == key_bits
    hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, KB, KB, true>), g1, dim3(kMThreads), 0, st, a);
  else if (a.d.value_bits == 2)
    hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, 2, KB, false>), g1, dim3(kMThreads), 0, st, a);
  else if (a.d.value_bits == 3)
    hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, 3, KB, false>), g1, dim3(kMThreads), 0, st, a);
  else
    hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, 4, KB, false>), g1, dim3(kMThreads), 0, st, a);
}

template <int GQ, int D>
void launch_valu(const DecodeArgs& a, dim3 grid, hipStream_t st) {
  if (a.d.value_bits == 2)
    hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 2, D>), grid, dim3(kThreads), 0, st, a);
  else if (a.d.value_bits == 3)
    hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 3, D>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 4, D>), grid, dim3(kThreads), 0, st, a);
}

template <int GQ>
hipError_t launch_split(const DecodeArgs& a, dim3 grid, hipStream_t st) {
  if (!mfma_path(a.d)) {
    if (a.d.head_dim == 64)
      launch_valu<GQ, 64>(a, grid, st);
    else if (a.d.head_dim == 128)
      launch_valu<GQ, 128>(a, grid, st);
    else
      launch_valu<GQ, 256>(a, grid, st);
    return hipGetLastError();
  }
  // one-dimensional over (split, kv head, seq) items
  const dim3 g1(grid.x * grid.y * grid.z);
  if (a.d.key_bits == 4)
    launch_mfma_kb<GQ, 4>(a, g1, st);
  else if (a.d.key_bits == 3)
    launch_mfma_kb<GQ, 3>(a, g1, st);
  else
    launch_mfma_kb<GQ, 2>(a, g1, st);
  return hipGetLastError();
}

DecodeArgs make_args(const tqk_cache_desc* d, const tqk_cache_ptrs* p, const Plan& pl, int batch,
                     const void* q, const int32_t* seq_lens, const WsView& w) {
  const int ns = pl.n_cold_splits + pl.n_hot_splits;
  const size_t per = (size_t)batch * d->n_q_heads * ns;
  DecodeArgs a;
  a.d = *d;
  a.p = *p;
  a.q = q;
  a.seq_lens = seq_lens;
  a.arrive = w.arrive;
  a.pm = reinterpret_cast<float*>(w.partials);
  a.pl = a.pm + per;
  a.pacc = a.pl + per;
  a.n_cold_splits = pl.n_cold_splits;
  a.n_hot_splits = pl.n_hot_splits;
  a.groups_per_split = pl.groups_per_split;
  a.wave_blocks = pl.wave_blocks;
  a.hot_per_split = pl.hot_per_split;
  a.split_base = 0;
  a.batch = batch;
  a.reorder = mfma_path(*d) && (long)pl.n_cold_splits * d->n_kv_heads * batch > device_cus();
  a.out = nullptr;
  return a;
}

WsView caller_ws(const Plan& pl, void* ws) {
  return WsView{reinterpret_cast<uint32_t*>(ws), static_cast<char*>(ws) + pl.counter_bytes};
}

// Arguments every decode entry point validates the same way.
int check_decode_args(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int batch, int max_len) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || batch <= 0 || max_len <= 0) return TQK_EINVAL;
  if (d->key_grid == 2 && !p->knorm) return TQK_EINVAL;
  if (batch > counter_seqs(*d)) return TQK_EINVAL;
  return TQK_OK;
}

// The split kernel (validated arguments); `out` non-null selects the MFMA
// kernel's in-kernel merge.
int launch_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, const Plan& pl, int batch,
                  const void* q, const int32_t* seq_lens, const WsView& w, void* stream,
                  float* out) {
  DecodeArgs a = make_args(d, p, pl, batch, q, seq_lens, w);
  if (out && mfma_path(*d)) a.out = out;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // (the MFMA kernel's workgroups are the coded splits; each also covers a
  // share of the hot window)
  const dim3 grid(mfma_path(*d) ? pl.n_cold_splits : pl.n_cold_splits + pl.n_hot_splits,
                  d->n_kv_heads, batch);
  hipError_t e;
  // kernels exist for 1, 2, 4 and 8 query heads per kv head; other counts
  // run on the next larger one with zero-query padding heads
  switch (d->n_q_heads / d->n_kv_heads) {
    case 1: e = launch_split<1>(a, grid, st); break;
    case 2: e = launch_split<2>(a, grid, st); break;
    case 3: case 4: e = launch_split<4>(a, grid, st); break;
    case 5: case 6: case 7: case 8: e = launch_split<8>(a, grid, st); break;
    default: return TQK_EUNSUPPORTED;
  }
  return e == hipSuccess ? TQK_OK : TQK_EHIP;
}

// tqk_merge over the partials the split kernel left (validated arguments).
int launch_merge(const tqk_cache_desc* d, const tqk_cache_ptrs* p, const Plan& pl, int batch,
                 const WsView& w, float* out, float* m_out, float* l_out, float* acc_out,
                 void* stream) {
  const DecodeArgs a = make_args(d, p, pl, batch, nullptr, nullptr, w);
  MergeArgs m;
  m.pm = a.pm;
  m.pl = a.pl;
  m.pacc = a.pacc;
  m.pi = p->pi;
  m.n_cold_splits = pl.n_cold_splits;
  m.n_splits = pl.n_cold_splits + pl.n_hot_splits;
  m.n_q_heads = d->n_q_heads;
  m.n_kv_heads = d->n_kv_heads;
  m.out = out;
  m.m_out = m_out;
  m.l_out = l_out;
  m.acc_out = acc_out;
  const dim3 grid(d->n_kv_heads, batch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (d->head_dim == 64)
    hipLaunchKernelGGL(tqk_merge<64>, grid, dim3(128), 0, st, m);
  else if (d->head_dim == 128)
    hipLaunchKernelGGL(tqk_merge<128>, grid, dim3(256), 0, st, m);
  else
    hipLaunchKernelGGL(tqk_merge<256>, grid, dim3(512), 0, st, m);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int run_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int batch, const void* q,
               const int32_t* seq_lens, int max_len, void* ws, size_t ws_bytes, void* stream,
               float* out = nullptr) {
  int rc = check_decode_args(d, p, batch, max_len);
  if (rc != TQK_OK) return rc;
  if (!q || !seq_lens) return TQK_EINVAL;
  const Plan pl = make_plan(d, batch, max_len);
  if (!ws || ws_bytes < pl.ws_bytes) return TQK_EWORKSPACE;
  return launch_splits(d, p, pl, batch, q, seq_lens, caller_ws(pl, ws), stream, out);
}

int run_merge(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int batch, int max_len, float* out,
              float* m_out, float* l_out, float* acc_out, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_decode_args(d, p, batch, max_len);
  if (rc != TQK_OK) return rc;
  if (!out && !(m_out && l_out && acc_out)) return TQK_EINVAL;
  const Plan pl = make_plan(d, batch, max_len);
  if (!ws || ws_bytes < pl.ws_bytes) return TQK_EWORKSPACE;
  return launch_merge(d, p, pl, batch, caller_ws(pl, ws), out, m_out, l_out, acc_out, stream);
}

// ---- the no-allocation decode's scratch ------------------------------------
// One zero-fill kernel for the scratch array's counter region (a kernel, not
// hipMemsetAsync, so that no memset node is recorded if a caller captures it).
__global__ void tqk_zero_words(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

// Device scratch of tqk_decode_noalloc, one copy per GPU for the life of the
// process: kNoAllocCounters arrival counters, then the split partials.  The
// array's name is a host-side stand-in: host code only ever uses the address
// hipGetSymbolAddress returns for the current device (noalloc_scratch()).
constexpr int kNoAllocCounters = 1 << 16;         // (sequence, kv head) pairs per call
constexpr size_t kNoAllocBytes = (size_t)32 << 20;  // 32 MiB per GPU
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The current device's scratch address, resolved (and its counters zeroed,
// on `stream`) at the first call on that device.
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TQK_EHIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return TQK_EHIP;
    hipLaunchKernelGGL(tqk_zero_words, dim3(kNoAllocCounters / 256), dim3(256), 0, stream,
                       static_cast<uint32_t*>(ptr), kNoAllocCounters);
    if (hipGetLastError() != hipSuccess) return TQK_EHIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TQK_OK;
}

}  // namespace

extern "C" {

int tqk_version(void) { return 9; }

int tqk_check_desc(const tqk_cache_desc* d) {
  if (!d) return TQK_EINVAL;
  if (!head_dim_ok(d->head_dim)) return TQK_EUNSUPPORTED;
  if (d->input_f32 != 0 && d->input_f32 != 1) return TQK_EINVAL;
  if (d->key_bits < 2 || d->key_bits > 4) return TQK_EUNSUPPORTED;
  if (d->key_grid < 0 || d->key_grid > 2) return TQK_EINVAL;
  // NF4 is a 4-bit grid; 3- and 2-bit keys are uniform or PolarQuant
  if (d->key_bits != 4 && d->key_grid == 0) return TQK_EUNSUPPORTED;
  // PolarQuant keys share the value codebook and carry no side-list
  if (d->key_grid == 2 && (d->key_bits != d->value_bits || d->outliers_per_channel != 0)) return TQK_EUNSUPPORTED;
  if (d->value_bits < 2 || d->value_bits > 4) return TQK_EUNSUPPORTED;
  if (d->zero_point < 0 || d->zero_point > 2 || (d->zero_point != 0 && d->key_grid != 0))
    return TQK_EINVAL;
  if (d->n_kv_heads <= 0 || d->n_q_heads <= 0 || d->n_q_heads % d->n_kv_heads) return TQK_EINVAL;
  const int gq = d->n_q_heads / d->n_kv_heads;
  if (gq < 1 || gq > 8) return TQK_EUNSUPPORTED;
  if (d->hot_window < 1) return TQK_EINVAL;
  if (d->group_tokens != (d->hot_window + 1) / 2) return TQK_EINVAL;
  if (d->group_tokens < 1 || d->group_tokens > TQK_MAX_G) return TQK_EUNSUPPORTED;
  if (d->page_tokens < 1 || d->group_tokens % d->page_tokens) return TQK_EINVAL;
  if (d->hot_ring < d->hot_window) return TQK_EINVAL;
  if (d->outliers_per_channel < 0 || d->outlier_cap < 0) return TQK_EINVAL;
  if (d->max_groups_per_seq < 0 || d->max_pages_per_seq < 0 || d->n_pages < 1) return TQK_EINVAL;
  return TQK_OK;
}

size_t tqk_decode_workspace_bytes(const tqk_cache_desc* d, int32_t batch, int32_t max_len) {
  if (!d || batch <= 0 || max_len <= 0 || batch > counter_seqs(*d)) return 0;
  return make_plan(d, batch, max_len).ws_bytes;
}

int tqk_decode(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
               const void* q, const int32_t* seq_lens, int32_t max_len, float* out,
               void* workspace, size_t workspace_bytes, void* stream) {
  if (!out) return TQK_EINVAL;
  int rc = run_splits(d, p, batch, q, seq_lens, max_len, workspace, workspace_bytes, stream, out);
  if (rc != TQK_OK) return rc;
  // the MFMA kernel merged in its last workgroups
  if (mfma_path(*d)) return TQK_OK;
  return run_merge(d, p, batch, max_len, out, nullptr, nullptr, nullptr, workspace,
                   workspace_bytes, stream);
}

int tqk_decode_noalloc(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                       const void* q, const int32_t* seq_lens, int32_t max_len, float* out,
                       void* stream) {
  int rc = check_decode_args(d, p, batch, max_len);
  if (rc != TQK_OK) return rc;
  if (!q || !seq_lens || !out) return TQK_EINVAL;
  const Plan pl = make_plan(d, batch, max_len);
  constexpr size_t kCounterBytes = (size_t)kNoAllocCounters * sizeof(uint32_t);
  if ((size_t)batch * d->n_kv_heads > (size_t)kNoAllocCounters ||
      pl.partial_bytes > kNoAllocBytes - kCounterBytes)
    return TQK_EWORKSPACE;
  void* base = nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  rc = noalloc_scratch(st, &base);
  if (rc != TQK_OK) return rc;
  const WsView w{static_cast<uint32_t*>(base), static_cast<char*>(base) + kCounterBytes};
  rc = launch_splits(d, p, pl, batch, q, seq_lens, w, stream, out);
  if (rc != TQK_OK || mfma_path(*d)) return rc;
  return launch_merge(d, p, pl, batch, w, out, nullptr, nullptr, nullptr, stream);
}

int tqk_decode_partials(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                        const void* q, const int32_t* seq_lens, int32_t max_len,
                        float* m, float* l, float* acc, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (!m || !l || !acc) return TQK_EINVAL;
  int rc = run_splits(d, p, batch, q, seq_lens, max_len, workspace, workspace_bytes, stream);
  if (rc != TQK_OK) return rc;
  return run_merge(d, p, batch, max_len, nullptr, m, l, acc, workspace, workspace_bytes, stream);
}

int tqk_decode_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                      const void* q, const int32_t* seq_lens, int32_t max_len,
                      void* workspace, size_t workspace_bytes, void* stream) {
  return run_splits(d, p, batch, q, seq_lens, max_len, workspace, workspace_bytes, stream);
}

int tqk_decode_merge(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                     int32_t max_len, float* out, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (!out) return TQK_EINVAL;
  return run_merge(d, p, batch, max_len, out, nullptr, nullptr, nullptr, workspace,
                   workspace_bytes, stream);
}

}  // extern "C"
