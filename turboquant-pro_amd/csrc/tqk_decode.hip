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
#include "tqk_common.h"

namespace {

struct DecodeArgs {
  tqk_cache_desc d;
  tqk_cache_ptrs p;
  const uint16_t* q;
  const int32_t* seq_lens;
  float* pm;    // [batch][Hq][n_splits]
  float* pl;    // [batch][Hq][n_splits]
  float* pacc;  // [batch][Hq][n_splits][D]
  int n_cold_splits;
  int n_hot_splits;
  int groups_per_split;
  int hot_per_split;
  int split_base;  // added to blockIdx.x (hot-only launches start after the coded splits)
};

struct MergeArgs {
  const float* pm;
  const float* pl;
  const float* pacc;
  const float* pi;
  int n_cold_splits;
  int n_splits;
  int n_q_heads;
  float* out;       // normalised output, or nullptr
  float* m_out;     // partial-state outputs (when out == nullptr)
  float* l_out;
  float* acc_out;
};

constexpr int kThreads = 256;

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

template <int GQ, int VB>
__global__ __launch_bounds__(kThreads) void tqk_decode_split_valu(DecodeArgs a) {
  constexpr int D = TQK_D;
  constexpr int VROW = D * VB / 8;
  const int split = blockIdx.x + a.split_base, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const tqk_cache_desc& d = a.d;
  const int Hkv = d.n_kv_heads, Hq = d.n_q_heads, G = d.group_tokens, P = d.page_tokens;
  const int L = a.seq_lens[b];
  const int ng = n_groups_of(L, d.hot_window, G);
  const int n_cold = ng * G;
  const float sm = d.sm_scale;

  __shared__ float q_s[GQ][D];
  __shared__ float w_s[GQ][D];
  __shared__ float sc_s[GQ][kThreads];
  __shared__ float kl_s[256][2];
  __shared__ float vl_s[(VB == 3) ? 64 : 256][2];
  __shared__ float red_s[4][GQ];
  __shared__ float a_s[D], mu_s[D];
  __shared__ float accr_s[4][GQ][D];

  for (int i = tid; i < GQ * D; i += kThreads)
    q_s[i / D][i % D] = h2f(a.q[((size_t)b * Hq + h * GQ + i / D) * D + i % D]);
  kl_s[tid][0] = kNF4[rev4(tid >> 4)];
  kl_s[tid][1] = kNF4[rev4(tid & 15)];
  if (VB == 3) {
    if (tid < 64) {
      vl_s[tid][0] = a.p.vcent[tid & 7];
      vl_s[tid][1] = a.p.vcent[tid >> 3];
    }
  } else {
    vl_s[tid & 255][0] = a.p.vcent[tid & 15];
    vl_s[tid & 255][1] = a.p.vcent[(tid >> 4) & 15];
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

  const int jp = tid & 63, tq = tid >> 6;
  const int32_t* __restrict__ bt = a.p.block_table;

  if (split < a.n_cold_splits) {
    const int g0 = split * a.groups_per_split;
    const int g1 = min(ng, g0 + a.groups_per_split);
    for (int g = g0; g < g1; ++g) {
      const int slot = a.p.group_table[(size_t)b * d.max_groups_per_seq + g];
      const size_t mbase = ((size_t)slot * Hkv + h) * D;
      if (tid < D) {
        const float av = a.p.gscale[mbase + tid];
        const float mv = a.p.gmean[mbase + tid];
        a_s[tid] = av;
        mu_s[tid] = mv;
        float bias_part[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          w_s[i][tid] = q_s[i][tid] * av;
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
      for (int i = 0; i < GQ; ++i) bias[i] = red_s[0][i] + red_s[1][i];
      __syncthreads();

      // dense key scores: one token per thread
      float norm_t = 0.f;
      if (tid < G) {
        const size_t row = page_row(bt, d.max_pages_per_seq, b, g * G + tid, P, Hkv, h);
        const uint4* kr = reinterpret_cast<const uint4*>(a.p.kcodes + row * (D / 2));
        float s[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) s[i] = 0.f;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const uint4 w4 = kr[c4];
          const uint32_t wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
              const uint32_t byte = (wv[wi] >> (8 * bi)) & 0xFFu;
              const int j = (c4 * 16 + wi * 4 + bi) * 2;
              const float k0 = kl_s[byte][0], k1 = kl_s[byte][1];
#pragma unroll
              for (int i = 0; i < GQ; ++i) s[i] += w_s[i][j] * k0 + w_s[i][j + 1] * k1;
            }
          }
        }
#pragma unroll
        for (int i = 0; i < GQ; ++i) sc_s[i][tid] = (s[i] + bias[i]) * sm;
        norm_t = a.p.vnorm[row];
      }
      __syncthreads();

      // sparse outlier corrections: q_j * (val - dense) added to token rows
      const size_t obase = (size_t)slot * Hkv + h;
      const int no = min(a.p.ocount[obase * TQK_NOB + TQK_NOB - 1], d.outlier_cap);
      for (int e = tid; e < no; e += kThreads) {
        const uint32_t ent = a.p.oent[obase * d.outlier_cap + e];
        const int pos = ent & 0xFFFFu;
        const float val = h2f((uint16_t)(ent >> 16));
        const int tt = pos >> 7, j = pos & (D - 1);
        const size_t row = page_row(bt, d.max_pages_per_seq, b, g * G + tt, P, Hkv, h);
        const uint32_t byte = a.p.kcodes[row * (D / 2) + (j >> 1)];
        const uint32_t c = (j & 1) ? rev4(byte & 15u) : rev4(byte >> 4);
        const float delta = val - (a_s[j] * kNF4[c] + mu_s[j]);
#pragma unroll
        for (int i = 0; i < GQ; ++i) atomicAdd(&sc_s[i][tt], q_s[i][j] * delta * sm);
      }
      __syncthreads();

      softmax_update<GQ>(sc_s, G, m_run, l_run, acc0, acc1, red_s, norm_t);

      // value accumulation in rotated code space: thread = (channel pair, token quarter)
      const int tend = min(G, tq * 64 + 64);
      for (int tt = tq * 64; tt < tend; ++tt) {
        const size_t row = page_row(bt, d.max_pages_per_seq, b, g * G + tt, P, Hkv, h);
        uint32_t f;
        if (VB == 3) {
          const uint32_t* vr = reinterpret_cast<const uint32_t*>(a.p.vcodes + row * VROW);
          const int bit = 6 * jp, wd = bit >> 5, sh = bit & 31;
          const uint32_t lo = vr[wd];
          const uint32_t hi = (sh > 26) ? vr[wd + 1] : 0u;
          f = (uint32_t)(((((uint64_t)hi) << 32) | lo) >> sh) & 63u;
        } else {
          f = a.p.vcodes[row * VROW + jp];
        }
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
    // fp16 hot window slice
    const int hs = split - a.n_cold_splits;
    const int t0 = n_cold + hs * a.hot_per_split;
    const int t1 = min(L, t0 + a.hot_per_split);
    if (t0 < t1) {
      const int n = t1 - t0;
      const int R = d.hot_ring;
      const size_t hbase = ((size_t)b * Hkv + h) * R;
      if (tid < n) {
        const uint4* kr = reinterpret_cast<const uint4*>(a.p.hot_k + (hbase + (t0 + tid) % R) * D);
        float s[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i) s[i] = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
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
#pragma unroll
        for (int i = 0; i < GQ; ++i) sc_s[i][tid] = s[i] * sm;
      }
      __syncthreads();
      softmax_update<GQ>(sc_s, n, m_run, l_run, acc0, acc1, red_s, 1.0f);
      const int tend = min(n, tq * 64 + 64);
      for (int tt = tq * 64; tt < tend; ++tt) {
        const uint32_t two =
            reinterpret_cast<const uint32_t*>(a.p.hot_v + (hbase + (t0 + tt) % R) * D)[jp];
        const float c0 = h2f((uint16_t)(two & 0xFFFFu)), c1 = h2f((uint16_t)(two >> 16));
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
          const float pp = sc_s[i][tt];
          acc0[i] += pp * c0;
          acc1[i] += pp * c1;
        }
      }
    }
  }

  // combine the four token quarters and write the split's state
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    accr_s[tq][i][2 * jp] = acc0[i];
    accr_s[tq][i][2 * jp + 1] = acc1[i];
  }
  __syncthreads();
  const int ns = a.n_cold_splits + a.n_hot_splits;
  for (int x = tid; x < GQ * D; x += kThreads) {
    const int i = x / D, j = x % D;
    const float s4 = (accr_s[0][i][j] + accr_s[1][i][j]) + (accr_s[2][i][j] + accr_s[3][i][j]);
    a.pacc[(((size_t)b * Hq + h * GQ + i) * ns + split) * D + j] = s4;
  }
#pragma unroll
  for (int i = 0; i < GQ; ++i) {
    if (tid == i) {
      const size_t o = ((size_t)b * Hq + h * GQ + i) * ns + split;
      a.pm[o] = m_run[i];
      a.pl[o] = l_run[i];
    }
  }
}


// ---------------------------------------------------------------------------
// MFMA split kernel for coded groups (value codes in the tiled order).
//
// One wave owns one group at a time and walks it in 32-token blocks:
//   QK^T  C[token][col] += A[token][ch] * B[ch][col]   (v_mfma_f32_16x16x32_f16)
//         A = NF4 level of the key code, split fp16 hi + lo (two MFMAs),
//         B = q * nf4_scale split fp16 hi (cols 0..GQ-1) + lo (cols GQ..2GQ-1);
//         col h + col h+GQ is the full-precision score of query head h.
//   PV    O[row][ch] += P[row][token] * V[token][ch]
//         P = softmax weight * value norm, hi rows 0..GQ-1, lo rows GQ..2GQ-1,
//         V = value centroid split fp16 hi + lo (two MFMAs).
// The QK^T output layout (lane = 16*lg + col holds tokens 4lg..4lg+3) is the
// PV A-operand layout, so scores never leave registers except for the sparse
// outlier corrections, which go through a per-wave LDS block.
// Key bytes and value fields are turned into fp16 hi/lo operand pairs through
// a bank-replicated LDS table (16 copies, one per lane of a 16-lane LDS pass).
// ---------------------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
union H8 {
  half8_t h;
  uint32_t u[4];
};

constexpr int kLutEntry = 256;   // bytes per table entry: 16 key copies | 16 value copies
constexpr int kLutV = 128;       // value copies start here inside an entry

__device__ __forceinline__ uint2 split_pair(float x0, float x1) {
  const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
  const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
  return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                    (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16));
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS address of key-table entry (byte k of word x), copy offset in `off` (< 256):
// one v_perm_b32: byte 1 <- x.byte[k], byte 0 <- off.byte[0], bytes 2..3 <- 0.
template <int K>
__device__ __forceinline__ uint32_t lut_addr_byte(uint32_t x, uint32_t off) {
  return __builtin_amdgcn_perm(x, off, 0x0C0C0000u | ((4u + K) << 8));
}

// 6-bit field m of a 96-bit value-code unit (3-bit codes).
template <int M>
__device__ __forceinline__ uint32_t v3_field(uint32_t u0, uint32_t u1, uint32_t u2) {
  if constexpr (M <= 9) {
    const uint64_t lo = (uint64_t)u0 | ((uint64_t)u1 << 32);
    return (uint32_t)(lo >> (6 * M)) & 63u;
  } else {
    const uint64_t hi = (uint64_t)u1 | ((uint64_t)u2 << 32);
    return (uint32_t)(hi >> (6 * M - 32)) & 63u;
  }
}

template <int GQ, int VB>
__global__ __launch_bounds__(kThreads, 2) void tqk_decode_split_mfma(DecodeArgs a) {
  constexpr int D = TQK_D;
  constexpr int VROW = D * VB / 8;
  constexpr int UNIT = VROW / 4;
  constexpr int NCOL = 2 * GQ;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lg = lane >> 4, c = lane & 15;
  const tqk_cache_desc& d = a.d;
  const int Hkv = d.n_kv_heads, Hq = d.n_q_heads, G = d.group_tokens, P = d.page_tokens;
  const int L = a.seq_lens[b];
  const int ng = n_groups_of(L, d.hot_window, G);
  const float sm = d.sm_scale;

  __shared__ __align__(16) uint8_t lut[256 * kLutEntry];
  __shared__ float q_s[GQ][D];
  __shared__ float am_s[4][2][D];
  __shared__ float sc_s[4][32][GQ];

  {
    const int e = tid;
    const uint2 kv = split_pair(kNF4[rev4((uint32_t)e >> 4)], kNF4[rev4((uint32_t)e & 15u)]);
    uint2 vv = make_uint2(0u, 0u);
    if (e < (1 << (2 * VB))) {
      const int m = (1 << VB) - 1;
      vv = split_pair(a.p.vcent[e & m], a.p.vcent[e >> VB]);
    }
    uint8_t* ent = lut + e * kLutEntry;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      *reinterpret_cast<uint2*>(ent + q * 8) = kv;
      *reinterpret_cast<uint2*>(ent + kLutV + q * 8) = vv;
    }
  }
  for (int i = tid; i < GQ * D; i += kThreads)
    q_s[i / D][i % D] = h2f(a.q[((size_t)b * Hq + h * GQ + i / D) * D + i % D]);
  __syncthreads();

  const int hcol = c % GQ;
  const bool active = c < NCOL, is_hi = c < GQ;
  const uint32_t koff = (uint32_t)c * 8u, voff = (uint32_t)kLutV + (uint32_t)c * 8u;
  const int32_t* __restrict__ bt = a.p.block_table;
  const uint8_t* __restrict__ kcodes = a.p.kcodes;
  const uint8_t* __restrict__ vcodes = a.p.vcodes;
  const float* __restrict__ vnorm = a.p.vnorm;

  float m_run = -INFINITY, l_run = 0.f;
  floatx4_t O[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) O[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const int g0 = split * a.groups_per_split;
  const int g1 = min(ng, g0 + a.groups_per_split);
  for (int g = g0 + w; g < g1; g += 4) {
    const int slot = a.p.group_table[(size_t)b * d.max_groups_per_seq + g];
    const size_t mbase = ((size_t)slot * Hkv + h) * D;
    {
      const float2 av = reinterpret_cast<const float2*>(a.p.gscale + mbase)[lane];
      const float2 mv = reinterpret_cast<const float2*>(a.p.gmean + mbase)[lane];
      am_s[w][0][2 * lane] = av.x;
      am_s[w][0][2 * lane + 1] = av.y;
      am_s[w][1][2 * lane] = mv.x;
      am_s[w][1][2 * lane + 1] = mv.y;
    }
    wave_sync();
    // B operand of QK^T: channel 32*lg + 8*ks + e, column c
    H8 Bw[4];
    float biasp = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int ch = 32 * lg + 8 * ks + e;
        const float qv = q_s[hcol][ch];
        const float wv = qv * am_s[w][0][ch];
        const _Float16 hi = (_Float16)wv;
        const _Float16 lo = (_Float16)(wv - (float)hi);
        Bw[ks].h[e] = active ? (is_hi ? hi : lo) : (_Float16)0.f;
        biasp += qv * am_s[w][1][ch];
      }
    }
    biasp += __shfl_xor(biasp, 16, 64);
    biasp += __shfl_xor(biasp, 32, 64);
    const float bias = biasp;
    const size_t obase = (size_t)slot * Hkv + h;
    const int32_t* __restrict__ ob = a.p.ocount + obase * TQK_NOB;
    const uint32_t* __restrict__ oent = a.p.oent + obase * d.outlier_cap;

    const int nblk = G / 32;
    for (int blk = 0; blk < nblk; ++blk) {
      const int t0 = g * G + 32 * blk;
      const size_t rowA = page_row(bt, d.max_pages_per_seq, b, t0, P, Hkv, h);
      const size_t rowB = page_row(bt, d.max_pages_per_seq, b, t0 + 16, P, Hkv, h);
      const uint4 kA = *reinterpret_cast<const uint4*>(kcodes + (rowA + c) * (D / 2) + 16 * lg);
      const uint4 kB = *reinterpret_cast<const uint4*>(kcodes + (rowB + c) * (D / 2) + 16 * lg);
      uint32_t uA[UNIT / 4], uB[UNIT / 4];
      {
        const uint32_t* pA = reinterpret_cast<const uint32_t*>(vcodes + rowA * VROW + (16 * lg + c) * UNIT);
        const uint32_t* pB = reinterpret_cast<const uint32_t*>(vcodes + rowB * VROW + (16 * lg + c) * UNIT);
#pragma unroll
        for (int k = 0; k < UNIT / 4; ++k) {
          uA[k] = pA[k];
          uB[k] = pB[k];
        }
      }
      const float4 nA = *reinterpret_cast<const float4*>(vnorm + rowA + 4 * lg);
      const float4 nB = *reinterpret_cast<const float4*>(vnorm + rowB + 4 * lg);

      // ---- QK^T
      floatx4_t CA = {0.f, 0.f, 0.f, 0.f}, CB = {0.f, 0.f, 0.f, 0.f};
      const uint32_t kwA[4] = {kA.x, kA.y, kA.z, kA.w};
      const uint32_t kwB[4] = {kB.x, kB.y, kB.z, kB.w};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        H8 ah, al, bh, bl;
        uint2 t;
#define TQK_KLOAD(K)                                                                 \
  t = *reinterpret_cast<const uint2*>(lut + lut_addr_byte<K>(kwA[ks], koff));        \
  ah.u[K] = t.x;                                                                     \
  al.u[K] = t.y;                                                                     \
  t = *reinterpret_cast<const uint2*>(lut + lut_addr_byte<K>(kwB[ks], koff));        \
  bh.u[K] = t.x;                                                                     \
  bl.u[K] = t.y;
        TQK_KLOAD(0)
        TQK_KLOAD(1)
        TQK_KLOAD(2)
        TQK_KLOAD(3)
#undef TQK_KLOAD
        CA = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah.h, Bw[ks].h, CA, 0, 0, 0);
        CA = __builtin_amdgcn_mfma_f32_16x16x32_f16(al.h, Bw[ks].h, CA, 0, 0, 0);
        CB = __builtin_amdgcn_mfma_f32_16x16x32_f16(bh.h, Bw[ks].h, CB, 0, 0, 0);
        CB = __builtin_amdgcn_mfma_f32_16x16x32_f16(bl.h, Bw[ks].h, CB, 0, 0, 0);
      }
      float s[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = (CA[i] + __shfl_xor(CA[i], GQ, 64) + bias) * sm;
        s[4 + i] = (CB[i] + __shfl_xor(CB[i], GQ, 64) + bias) * sm;
      }

      // ---- sparse outliers of this block: q_j * (val - dense) through LDS
      const int e0 = min(blk == 0 ? 0 : ob[blk - 1], d.outlier_cap);
      const int e1 = min(ob[blk], d.outlier_cap);
      if (e1 > e0) {
        if (c < GQ) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sc_s[w][4 * lg + i][c] = s[i];
            sc_s[w][16 + 4 * lg + i][c] = s[4 + i];
          }
        }
        wave_sync();
        for (int e = e0 + lane; e < e1; e += 64) {
          const uint32_t ent = oent[e];
          const int pos = ent & 0xFFFFu;
          const float val = h2f((uint16_t)(ent >> 16));
          const int bt_ = (pos >> 7) - 32 * blk, j = pos & (D - 1);
          const size_t row = (bt_ < 16) ? rowA + bt_ : rowB + (bt_ - 16);
          const uint32_t byte = kcodes[row * (D / 2) + (j >> 1)];
          const uint32_t code = (j & 1) ? rev4(byte & 15u) : rev4(byte >> 4);
          const float delta = (val - (am_s[w][0][j] * kNF4[code] + am_s[w][1][j])) * sm;
#pragma unroll
          for (int hh = 0; hh < GQ; ++hh) atomicAdd(&sc_s[w][bt_][hh], q_s[hh][j] * delta);
        }
        wave_sync();
        if (active) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            s[i] = sc_s[w][4 * lg + i][hcol];
            s[4 + i] = sc_s[w][16 + 4 * lg + i][hcol];
          }
        }
        wave_sync();
      }

      // ---- online softmax for head hcol
      float bm = s[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) bm = fmaxf(bm, s[i]);
      bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m_run, bm);
      const float corr = __expf(m_run - mn);
      m_run = mn;
      float p[8], ps = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = __expf(s[i] - mn);
        ps += p[i];
      }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      l_run = l_run * corr + ps;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ci = __shfl(corr, 16 * lg + 4 * lg + i, 64);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) O[nt][i] *= ci;
      }
      // P operand rows: hi (c < GQ) / lo (GQ <= c < 2GQ) of p * norm
      H8 pa;
      {
        const float nv[8] = {nA.x, nA.y, nA.z, nA.w, nB.x, nB.y, nB.z, nB.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = p[e] * nv[e];
          const _Float16 hi = (_Float16)x;
          const _Float16 lo = (_Float16)(x - (float)hi);
          pa.h[e] = active ? (is_hi ? hi : lo) : (_Float16)0.f;
        }
      }
      // ---- PV over the 8 channel tiles (channel 8*c + nt)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        H8 vh, vl;
        uint32_t f[4];
        if constexpr (VB == 3) {
#define TQK_F3(M) (nt == (M) / 2 ? 0 : 0)
          switch (nt) {
#define TQK_V3CASE(NT)                                        \
  case NT:                                                    \
    f[0] = v3_field<2 * NT>(uA[0], uA[1], uA[2]);             \
    f[1] = v3_field<2 * NT + 1>(uA[0], uA[1], uA[2]);         \
    f[2] = v3_field<2 * NT>(uB[0], uB[1], uB[2]);             \
    f[3] = v3_field<2 * NT + 1>(uB[0], uB[1], uB[2]);         \
    break;
            TQK_V3CASE(0) TQK_V3CASE(1) TQK_V3CASE(2) TQK_V3CASE(3)
            TQK_V3CASE(4) TQK_V3CASE(5) TQK_V3CASE(6) TQK_V3CASE(7)
#undef TQK_V3CASE
#undef TQK_F3
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint2 t = *reinterpret_cast<const uint2*>(lut + ((f[k] << 8) | voff));
            vh.u[k] = t.x;
            vl.u[k] = t.y;
          }
        } else {
          // 4-bit: field m = byte m of the 16-byte unit
          const uint32_t wa = uA[nt >> 1], wb = uB[nt >> 1];
          const int k0 = 2 * (nt & 1);
          f[0] = (wa >> (8 * k0)) & 0xFFu;
          f[1] = (wa >> (8 * k0 + 8)) & 0xFFu;
          f[2] = (wb >> (8 * k0)) & 0xFFu;
          f[3] = (wb >> (8 * k0 + 8)) & 0xFFu;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint2 t = *reinterpret_cast<const uint2*>(lut + ((f[k] << 8) | voff));
            vh.u[k] = t.x;
            vl.u[k] = t.y;
          }
        }
        O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa.h, vh.h, O[nt], 0, 0, 0);
        O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa.h, vl.h, O[nt], 0, 0, 0);
      }
    }
  }

  // ---- combine the four waves' states (the table is no longer needed)
  __syncthreads();
  float* cm = reinterpret_cast<float*>(lut);  // [4][GQ]
  float* cl = cm + 4 * GQ;                    // [4][GQ]
  float* co = cl + 4 * GQ;                    // [4][GQ][D]
  if (lg == 0 && c < GQ) {
    cm[w * GQ + c] = m_run;
    cl[w * GQ + c] = l_run;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * lg + i;
    if (r < GQ) {
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) co[(w * GQ + r) * D + 8 * c + nt] = O[nt][i];
    }
  }
  wave_sync();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * lg + i;
    if (r >= GQ && r < NCOL) {
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) co[(w * GQ + r - GQ) * D + 8 * c + nt] += O[nt][i];
    }
  }
  __syncthreads();
  const int ns = a.n_cold_splits + a.n_hot_splits;
  for (int x = tid; x < GQ * D; x += kThreads) {
    const int i = x / D, j = x % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww)
      if (cl[ww * GQ + i] > 0.f) M = fmaxf(M, cm[ww * GQ + i]);
    float den = 0.f, acc = 0.f;
    if (M > -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float l = cl[ww * GQ + i];
        if (l > 0.f) {
          const float wt = __expf(cm[ww * GQ + i] - M);
          den += l * wt;
          acc += co[(ww * GQ + i) * D + j] * wt;
        }
      }
    }
    const size_t o = ((size_t)b * Hq + h * GQ + i) * ns + split;
    a.pacc[o * D + j] = acc;
    if (j == 0) {
      a.pm[o] = M;
      a.pl[o] = den;
    }
  }
}

// One workgroup per (query head, sequence), one thread per channel.
__global__ __launch_bounds__(TQK_D) void tqk_merge(MergeArgs a) {
  constexpr int D = TQK_D;
  const int qh = blockIdx.x, b = blockIdx.y, j = threadIdx.x;
  const size_t base = ((size_t)b * a.n_q_heads + qh) * a.n_splits;
  __shared__ float crot_s[D];
  float M = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s)
    if (a.pl[base + s] > 0.f) M = fmaxf(M, a.pm[base + s]);
  float den = 0.f, cr = 0.f, hr = 0.f;
  for (int s = 0; s < a.n_splits; ++s) {
    const float l = a.pl[base + s];
    if (l > 0.f) {
      const float w = __expf(a.pm[base + s] - M);
      den += l * w;
      const float v = a.pacc[(base + s) * D + j] * w;
      if (s < a.n_cold_splits) cr += v; else hr += v;
    }
  }
  crot_s[j] = cr;
  __syncthreads();
  float o = hr;
#pragma unroll 8
  for (int k = 0; k < D; ++k) o += crot_s[k] * a.pi[k * D + j];
  const size_t oi = ((size_t)b * a.n_q_heads + qh) * D + j;
  if (a.out) {
    a.out[oi] = o / den;
  } else {
    a.acc_out[oi] = o;
    if (j == 0) {
      a.m_out[(size_t)b * a.n_q_heads + qh] = M;
      a.l_out[(size_t)b * a.n_q_heads + qh] = den;
    }
  }
}

struct Plan {
  int n_cold_splits, n_hot_splits, groups_per_split, hot_per_split;
  size_t ws_bytes;
};

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
  if (v_tiled(G, d->page_tokens)) {
    // MFMA kernel: four waves per workgroup, each a run of groups
    int gpw = (int)((units + 4L * 1536 - 1) / (4L * 1536));
    if (gpw < 1) gpw = 1;
    gps = 4 * gpw;
  } else {
    gps = (int)((units + 4095) / 4096);
    if (gps < 1) gps = 1;
  }
  pl.groups_per_split = gps;
  pl.n_cold_splits = ngmax > 0 ? (ngmax + gps - 1) / gps : 0;
  const size_t ns = (size_t)(pl.n_cold_splits + pl.n_hot_splits);
  const size_t per = (size_t)batch * d->n_q_heads * ns;
  pl.ws_bytes = per * sizeof(float) * (2 + TQK_D) + 256;
  return pl;
}

template <int GQ>
hipError_t launch_split(const DecodeArgs& a, dim3 grid, hipStream_t st) {
  const bool tiled = v_tiled(a.d.group_tokens, a.d.page_tokens);
  if (!tiled) {
    if (a.d.value_bits == 3)
      hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 3>), grid, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 4>), grid, dim3(kThreads), 0, st, a);
    return hipGetLastError();
  }
  if (a.n_cold_splits > 0) {
    const dim3 gc(a.n_cold_splits, grid.y, grid.z);
    if (a.d.value_bits == 3)
      hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, 3>), gc, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((tqk_decode_split_mfma<GQ, 4>), gc, dim3(kThreads), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  DecodeArgs ah = a;
  ah.split_base = a.n_cold_splits;
  const dim3 gh(a.n_hot_splits, grid.y, grid.z);
  if (a.d.value_bits == 3)
    hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 3>), gh, dim3(kThreads), 0, st, ah);
  else
    hipLaunchKernelGGL((tqk_decode_split_valu<GQ, 4>), gh, dim3(kThreads), 0, st, ah);
  return hipGetLastError();
}

DecodeArgs make_args(const tqk_cache_desc* d, const tqk_cache_ptrs* p, const Plan& pl, int batch,
                     const uint16_t* q, const int32_t* seq_lens, void* ws) {
  const int ns = pl.n_cold_splits + pl.n_hot_splits;
  const size_t per = (size_t)batch * d->n_q_heads * ns;
  DecodeArgs a;
  a.d = *d;
  a.p = *p;
  a.q = q;
  a.seq_lens = seq_lens;
  a.pm = reinterpret_cast<float*>(ws);
  a.pl = a.pm + per;
  a.pacc = a.pl + per;
  a.n_cold_splits = pl.n_cold_splits;
  a.n_hot_splits = pl.n_hot_splits;
  a.groups_per_split = pl.groups_per_split;
  a.hot_per_split = pl.hot_per_split;
  a.split_base = 0;
  return a;
}

int run_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int batch, const uint16_t* q,
               const int32_t* seq_lens, int max_len, void* ws, size_t ws_bytes, void* stream) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || !q || !seq_lens || batch <= 0 || max_len <= 0) return TQK_EINVAL;
  const Plan pl = make_plan(d, batch, max_len);
  if (!ws || ws_bytes < pl.ws_bytes) return TQK_EWORKSPACE;
  const DecodeArgs a = make_args(d, p, pl, batch, q, seq_lens, ws);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(pl.n_cold_splits + pl.n_hot_splits, d->n_kv_heads, batch);
  hipError_t e;
  switch (d->n_q_heads / d->n_kv_heads) {
    case 1: e = launch_split<1>(a, grid, st); break;
    case 2: e = launch_split<2>(a, grid, st); break;
    case 4: e = launch_split<4>(a, grid, st); break;
    case 8: e = launch_split<8>(a, grid, st); break;
    default: return TQK_EUNSUPPORTED;
  }
  return e == hipSuccess ? TQK_OK : TQK_EHIP;
}

int run_merge(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int batch, int max_len, float* out,
              float* m_out, float* l_out, float* acc_out, void* ws, size_t ws_bytes, void* stream) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || batch <= 0 || max_len <= 0) return TQK_EINVAL;
  if (!out && !(m_out && l_out && acc_out)) return TQK_EINVAL;
  const Plan pl = make_plan(d, batch, max_len);
  if (!ws || ws_bytes < pl.ws_bytes) return TQK_EWORKSPACE;
  const DecodeArgs a = make_args(d, p, pl, batch, nullptr, nullptr, ws);
  MergeArgs m;
  m.pm = a.pm;
  m.pl = a.pl;
  m.pacc = a.pacc;
  m.pi = p->pi;
  m.n_cold_splits = pl.n_cold_splits;
  m.n_splits = pl.n_cold_splits + pl.n_hot_splits;
  m.n_q_heads = d->n_q_heads;
  m.out = out;
  m.m_out = m_out;
  m.l_out = l_out;
  m.acc_out = acc_out;
  hipLaunchKernelGGL(tqk_merge, dim3(d->n_q_heads, batch), dim3(TQK_D), 0,
                     reinterpret_cast<hipStream_t>(stream), m);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

}  // namespace

extern "C" {

int tqk_version(void) { return 1; }

int tqk_check_desc(const tqk_cache_desc* d) {
  if (!d) return TQK_EINVAL;
  if (d->head_dim != TQK_D) return TQK_EUNSUPPORTED;
  if (d->key_bits != 4) return TQK_EUNSUPPORTED;
  if (d->value_bits != 3 && d->value_bits != 4) return TQK_EUNSUPPORTED;
  if (d->n_kv_heads <= 0 || d->n_q_heads <= 0 || d->n_q_heads % d->n_kv_heads) return TQK_EINVAL;
  const int gq = d->n_q_heads / d->n_kv_heads;
  if (gq != 1 && gq != 2 && gq != 4 && gq != 8) return TQK_EUNSUPPORTED;
  if (d->hot_window < 1) return TQK_EINVAL;
  if (d->group_tokens != (d->hot_window + 1) / 2) return TQK_EINVAL;
  if (d->group_tokens < 1 || d->group_tokens > TQK_MAX_G) return TQK_EUNSUPPORTED;
  if (d->page_tokens < 1 || d->group_tokens % d->page_tokens) return TQK_EINVAL;
  if (d->hot_ring < d->hot_window) return TQK_EINVAL;
  if (d->outliers_per_channel < 0 || d->outlier_cap < 0) return TQK_EINVAL;
  if (d->max_groups_per_seq < 0 || d->max_pages_per_seq < 0) return TQK_EINVAL;
  return TQK_OK;
}

size_t tqk_decode_workspace_bytes(const tqk_cache_desc* d, int32_t batch, int32_t max_len) {
  if (!d || batch <= 0 || max_len <= 0) return 0;
  return make_plan(d, batch, max_len).ws_bytes;
}

int tqk_decode(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
               const uint16_t* q, const int32_t* seq_lens, int32_t max_len, float* out,
               void* workspace, size_t workspace_bytes, void* stream) {
  if (!out) return TQK_EINVAL;
  int rc = run_splits(d, p, batch, q, seq_lens, max_len, workspace, workspace_bytes, stream);
  if (rc != TQK_OK) return rc;
  return run_merge(d, p, batch, max_len, out, nullptr, nullptr, nullptr, workspace,
                   workspace_bytes, stream);
}

int tqk_decode_partials(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                        const uint16_t* q, const int32_t* seq_lens, int32_t max_len,
                        float* m, float* l, float* acc, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (!m || !l || !acc) return TQK_EINVAL;
  int rc = run_splits(d, p, batch, q, seq_lens, max_len, workspace, workspace_bytes, stream);
  if (rc != TQK_OK) return rc;
  return run_merge(d, p, batch, max_len, nullptr, m, l, acc, workspace, workspace_bytes, stream);
}

int tqk_decode_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                      const uint16_t* q, const int32_t* seq_lens, int32_t max_len,
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
