// Quantize-on-flush, hot-ring append and group reconstruction (gfx950).
//
// Bit-exactness contract (this file is compiled with -ffp-contract=off and
// uses explicitly rounded __f*_rn operations): every code, scale, mean, norm
// and outlier entry equals what the reference's NumPy encoder produces for the
// same fp16 inputs.  NumPy's operation order is restated exactly:
//   keys   (turboquant_pro/per_channel_kv.py:269-401, nf4_asym)
//     mean  = token-order sequential fp32 sum / G ("calibrated"; "sparse"
//             multiplies it by the DC-channel mask, "bias" takes it given)
//     amax  = max(max_s |x_s - mean|, 1e-8)            (NaN propagates)
//     cent  = mean + amax * NF4[l]
//     code  = first argmin_l |x - cent_l|               (NaN counts as minimal)
//     outlier threshold = k-th largest |x| (ties kept), flat (s, j) order
//   values (turboquant_pro/core.py:569-606, CPU full-QR branch)
//     norm  = sqrt(pairwise sum of squares)              (numpy pairwise_sum, n = D)
//     u     = v / max(norm, 1e-30)
//     y_e   = sequential over d of (u_d * PiT[d][e]), separately rounded
//     code  = #{ boundaries < y_e }                      (searchsorted, side="left";
//                                                         a NaN y_e takes the last code)
#include "tqk_common.h"

namespace {

constexpr int kThreads = 256;
// the group encode: four waves; its LDS (under 80 KiB) lets two workgroups share
// a CU, so one's latency-bound key phase runs beside the other's value rotation
constexpr int kEncThreads = 256;
constexpr int kEncWaves = kEncThreads / 64;

struct EncodeArgs {
  tqk_cache_desc d;
  tqk_cache_ptrs p;
  const int32_t* items;
  const int32_t* prev_len;
  const void* chunk_k;  // fp16, or fp32 (input_f32)
  const void* chunk_v;
  int chunk_tokens;
  int32_t* overflow;
};

// Source row (D values of type T: fp16 bits or fp32) of token t of sequence
// b, kv head h: the hot ring for tokens already in the cache, the appended
// chunk for new ones.
template <int D, typename T = uint16_t>
__device__ __forceinline__ const T* token_src(const EncodeArgs& a, const void* ring,
                                              const void* chunk, int b, int h, int t) {
  const tqk_cache_desc& d = a.d;
  const int prev = a.prev_len[b];
  if (t < prev)
    return static_cast<const T*>(ring) +
           (((size_t)b * d.n_kv_heads + h) * d.hot_ring + (t % d.hot_ring)) * D;
  return static_cast<const T*>(chunk) + (((size_t)b * d.n_kv_heads + h) * a.chunk_tokens + (t - prev)) * D;
}

__device__ __forceinline__ uint32_t abs_h(uint16_t x) { return x & 0x7FFFu; }

typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

// v into the K-long descending lists held in the two halves of t (one
// packed 16-bit max and min per list entry)
template <int K>
__device__ __forceinline__ void topk_insert(u16x2_t (&t)[K], u16x2_t v) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const u16x2_t hi = __builtin_elementwise_max(t[i], v);
    v = __builtin_elementwise_min(t[i], v);
    t[i] = hi;
  }
}

// The k-th largest (1 <= k <= K) of a channel's magnitude patterns, held two
// per register in m by the four lanes l, l ^ 16, l ^ 32, l ^ 48: each lane
// keeps the K largest of each half of its registers, the halves' lists are
// merged, then the lanes' lists over the two permlane swaps.  The largest T
// with #{m >= T} >= k is exactly this k-th largest value (with multiplicity),
// so it equals the bitwise threshold search's result.
template <int K>
__device__ __forceinline__ uint32_t kth_largest(const u16x2_t (&m)[TQK_MAX_G / 8], int k) {
  u16x2_t t[K];
#pragma unroll
  for (int i = 0; i < K; ++i) t[i] = u16x2_t{0, 0};
#pragma unroll
  for (int i = 0; i < TQK_MAX_G / 8; ++i) topk_insert<K>(t, m[i]);
  {
    u16x2_t sw[K];
#pragma unroll
    for (int i = 0; i < K; ++i) sw[i] = t[i].yx;
#pragma unroll
    for (int i = 0; i < K; ++i) topk_insert<K>(t, sw[i]);
  }
  // a permlane swap returns this lane's list and its partner's, in an order
  // that depends on the lane; the merge is symmetric in the two
#pragma unroll
  for (int step = 0; step < 2; ++step) {
    u16x2_t other[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const uint32_t x = __builtin_bit_cast(uint32_t, t[i]);
      const auto r = step == 0 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                               : __builtin_amdgcn_permlane16_swap(x, x, false, false);
      t[i] = __builtin_bit_cast(u16x2_t, (uint32_t)r[0]);
      other[i] = __builtin_bit_cast(u16x2_t, (uint32_t)r[1]);
    }
#pragma unroll
    for (int i = 0; i < K; ++i) topk_insert<K>(t, other[i]);
  }
  uint32_t T = t[0].x;
#pragma unroll
  for (int i = 1; i < K; ++i)
    if (i == k - 1) T = t[i].x;
  return T;
}

// Sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows).
__device__ __forceinline__ int sum_quarters(int x) {
  auto a = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
  x = (int)(a[0] + a[1]);
  auto b = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
  return (int)(b[0] + b[1]);
}


template <int VB, int D>
__global__ __launch_bounds__(kEncThreads) void tqk_encode_group(EncodeArgs a) {
  const int item = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const tqk_cache_desc& d = a.d;
  const int b = a.items[2 * item], g = a.items[2 * item + 1];
  const int G = d.group_tokens, P = d.page_tokens, Hkv = d.n_kv_heads;
  const int slot = a.p.group_table[(size_t)b * d.max_groups_per_seq + g];
  const int kout = d.outliers_per_channel;
  const size_t mbase = ((size_t)slot * Hkv + h) * D;
  const size_t obase = (size_t)slot * Hkv + h;

  // Key tile (fp16 bits, rows padded against bank conflicts).  Its rows also
  // take the key codes: the codes of token t overwrite the first D / 2 bytes of
  // row t once the wave that owns the row has read it (kc_row).  Then the area
  // holds the value phase's codes (vc_s) and normalised rows (u_s).
  __shared__ __align__(16) uint16_t kt_s[TQK_MAX_G][D + 8];
  __shared__ float stat_s[D][2];             // per channel: (mean, amax) or (min, scale)
  // per channel: 0x8000 - the fp16 magnitude threshold T (so m + it has bit 15
  // set exactly when m >= T; 0 for a NaN T), read eight channels at a time by
  // the side-list scan
  __shared__ __align__(16) uint16_t tbias_s[D];
  __shared__ uint32_t omask_s[TQK_MAX_G][D / 32];  // channels of each token stored in the side-list
  __shared__ int32_t wsum_s[kEncWaves];
  auto kc_row = [&](int t) { return reinterpret_cast<uint8_t*>(&kt_s[t][0]); };
  uint8_t (*vc_s)[D] = reinterpret_cast<uint8_t (*)[D]>(&kt_s[0][0]);
  static_assert(TQK_MAX_G * (D + 8) * 2 >= TQK_MAX_G * D + 64 * D * 4, "value staging overflows the key tile");

  if (d.key_grid != 2) {
    // ---- stage the key tile ----------------------------------------------
    for (int idx = tid; idx < G * (D / 8); idx += kEncThreads) {
      const int t = idx / (D / 8), c = idx % (D / 8);
      const uint4* src =
          reinterpret_cast<const uint4*>(token_src<D>(a, a.p.hot_k, a.chunk_k, b, h, g * G + t));
      reinterpret_cast<uint4*>(&kt_s[t][0])[c] = src[c];
    }
    __syncthreads();

    // ---- per-channel statistics (thread j: channel j) ------------------------
    if (tid < D && d.key_grid == 1) {
      // uniform keys (turboquant_pro/per_channel_kv.py:303-306): channel min and
      // max over the tokens, scale = max(max - min, 1e-8) / (2^bits - 1) (NaN propagates)
      const int j = tid;
      float mn = h2f(kt_s[0][j]), mx = mn;
      bool nan = (mn != mn);
      for (int s = 1; s < G; ++s) {
        const float xv = h2f(kt_s[s][j]);
        nan |= (xv != xv);
        mn = fminf(mn, xv);
        mx = fmaxf(mx, xv);
      }
      const float rng = __fsub_rn(mx, mn);
      const float sc = nan ? __builtin_nanf("") : __fdiv_rn(fmaxf(rng, 1e-8f), (float)((1 << d.key_bits) - 1));
      if (nan) mn = __builtin_nanf("");
      stat_s[j][0] = mn;
      stat_s[j][1] = sc;
      a.p.gscale[mbase + j] = sc;
      a.p.gmean[mbase + j] = mn;
    } else if (tid < D) {
      const int j = tid;
      // the zero point (turboquant_pro/per_channel_kv.py:327-345)
      float mu;
      if (d.zero_point == 2) {
        // "bias": the RoPE-averaged k_proj bias of the group's positions
        mu = a.p.zp_mean[((size_t)g * Hkv + h) * D + j];
      } else {
        float acc = 0.0f;
        for (int s = 0; s < G; ++s) acc = __fadd_rn(acc, h2f(kt_s[s][j]));
        // np.mean divides the fp32 sum by an intp count: a float64 division, then fp32
        mu = (float)((double)acc / (double)G);
        // "sparse": the mean times the DC-channel mask (a float product, so a
        // non-DC channel gets a signed zero, or NaN from a NaN mean)
        if (d.zero_point == 1) mu = __fmul_rn(mu, ((d.dc_mask[j >> 5] >> (j & 31)) & 1u) ? 1.0f : 0.0f);
      }
      float amax = 0.0f;
      bool nan = (mu != mu);
      for (int s = 0; s < G; ++s) {
        const float dv = fabsf(__fsub_rn(h2f(kt_s[s][j]), mu));
        nan |= (dv != dv);
        amax = fmaxf(amax, dv);
      }
      amax = nan ? __builtin_nanf("") : fmaxf(amax, 1e-8f);
      stat_s[j][0] = mu;
      stat_s[j][1] = amax;
      a.p.gscale[mbase + j] = amax;
      a.p.gmean[mbase + j] = mu;
    }
    // ---- outlier thresholds: the k-th largest |x| of each channel as the
    // largest fp16 magnitude pattern T with #{ |x_s| >= T } >= k (NaN patterns
    // order above inf, as np.partition does).  Every thread, 16 channels per
    // wave and pass: lanes l, l ^ 16, l ^ 32, l ^ 48 take a quarter of the
    // tokens each, two magnitudes per register.  For k <= 8 the k largest are
    // kept directly (packed 16-bit max/min insertion); otherwise a bitwise
    // search, a candidate's count the carry bit of a packed 16-bit add,
    // summed over the four lanes.
    if (kout > 0 && kout < G) {
      const int part = lane >> 4;
      for (int j = 16 * wv + (lane & 15); j < D; j += 16 * kEncWaves) {
        u16x2_t m2[TQK_MAX_G / 8];
#pragma unroll
        for (int i = 0; i < TQK_MAX_G / 8; ++i) {
          // lane quarter `part` takes token pairs 8i + 2 part (rows 4 apart
          // fall on LDS banks 8 apart, so the four quarters never conflict);
          // tokens past G count as magnitude 0
          const int s = 8 * i + 2 * part;
          m2[i] = u16x2_t{(uint16_t)(s < G ? abs_h(kt_s[s][j]) : 0u),
                          (uint16_t)(s + 1 < G ? abs_h(kt_s[s + 1][j]) : 0u)};
        }
        uint32_t T = 0;
        if (kout <= 5) {
          T = kth_largest<5>(m2, kout);
        } else if (kout <= 8) {
          T = kth_largest<8>(m2, kout);
        } else {
          for (int bit = 14; bit >= 0; --bit) {
            const uint32_t cand = T | (1u << bit);
            // m + (0x8000 - cand) has bit 15 set exactly when m >= cand (m, cand < 2^15)
            const uint16_t bias = (uint16_t)(0x8000u - cand);
            const u16x2_t bv = {bias, bias};
            uint32_t acc = 0;  // two 16-bit counts
#pragma unroll
            for (int i = 0; i < TQK_MAX_G / 8; ++i)
              acc += (__builtin_bit_cast(uint32_t, (u16x2_t)(m2[i] + bv)) >> 15) & 0x00010001u;
            const int cnt = sum_quarters((int)((acc & 0xFFFFu) + (acc >> 16)));
            if (cnt >= kout) T = cand;
          }
        }
        // the scan compares magnitudes as floats, as the reference's mask
        // |x| >= t does: a NaN threshold selects nothing (bias 0)
        if (part == 0) tbias_s[j] = (uint16_t)(T > 0x7C00u ? 0u : 0x8000u - T);
      }
    }
    __syncthreads();

    // ---- outlier side-list in flat (token, channel) order, one token per
    // thread.  ocount holds cumulative counts at every TQK_OBLK-token boundary
    // of the group (entry TQK_NOB-1 = total), so a decode block finds its
    // entries without searching; omask_s records the stored (token, channel)
    // positions, whose codes become the grid's zero level below.
    if (kout > 0) {
      const bool all = kout >= G;
      // the token's outlier channels, eight at a time: magnitudes and biases
      // as packed 16-bit pairs, bit 15 of each half of m + bias is the test
      // m >= T; NaN magnitudes (m > 0x7C00, where m + 0x03FF reaches bit 15)
      // are never selected, as |x| >= t is false for them
      uint32_t om[D / 32];
#pragma unroll
      for (int k = 0; k < D / 32; ++k) om[k] = 0u;
      if (tid < G) {
#pragma unroll
        for (int c8 = 0; c8 < D / 8; ++c8) {
          const uint4 xw = *reinterpret_cast<const uint4*>(&kt_s[tid][8 * c8]);
          const uint4 bw = *reinterpret_cast<const uint4*>(&tbias_s[8 * c8]);
          const uint32_t xs[4] = {xw.x, xw.y, xw.z, xw.w}, bs[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u16x2_t m = __builtin_bit_cast(u16x2_t, xs[i] & 0x7FFF7FFFu);
            const uint32_t t = __builtin_bit_cast(uint32_t, (u16x2_t)(m + __builtin_bit_cast(u16x2_t, bs[i])));
            const uint32_t tn = __builtin_bit_cast(uint32_t, (u16x2_t)(m + u16x2_t{0x03FF, 0x03FF}));
            const uint32_t sel = t & ~tn;
            const uint32_t two = ((sel >> 15) & 1u) | ((sel >> 30) & 2u);  // channels 8c8 + 2i, + 1
            om[c8 >> 2] |= two << (8 * (c8 & 3) + 2 * i);
          }
        }
        if (all) {
#pragma unroll
          for (int k = 0; k < D / 32; ++k) om[k] = 0xFFFFFFFFu;
        }
      }
      int cnt = 0;
      if (tid < G) {
#pragma unroll
        for (int k = 0; k < D / 32; ++k) cnt += __builtin_popcount(om[k]);
      }
      // block exclusive scan of cnt
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      if (lane == 63) wsum_s[wv] = incl;
      __syncthreads();
      int wofs = 0;
      for (int w = 0; w < wv; ++w) wofs += wsum_s[w];
      int total = 0;
      for (int w = 0; w < kEncWaves; ++w) total += wsum_s[w];
      int off = wofs + incl - cnt;
      // token s = TQK_OBLK*k - 1 closes block k-1: its inclusive offset is the bound
      if (tid < G && ((tid + 1) % TQK_OBLK) == 0 && (tid + 1) / TQK_OBLK <= TQK_NOB)
        a.p.ocount[obase * TQK_NOB + (tid + 1) / TQK_OBLK - 1] = off + cnt;
      if (tid < TQK_NOB && TQK_OBLK * (tid + 1) > G) a.p.ocount[obase * TQK_NOB + tid] = total;
      if (tid < G) {
        // entries in channel order; those past the side-list's capacity are
        // dropped (and leave their codes alone)
#pragma unroll
        for (int k = 0; k < D / 32; ++k) {
          uint32_t w = om[k];
          while (w) {
            const int j = 32 * k + __builtin_ctz(w);
            w &= w - 1u;
            if (off < d.outlier_cap)
              a.p.oent[obase * d.outlier_cap + off] = (uint32_t)(tid * D + j) | ((uint32_t)kt_s[tid][j] << 16);
            else
              om[k] &= ~(1u << (j & 31));
            ++off;
          }
        }
#pragma unroll
        for (int k = 0; k < D / 32; ++k) omask_s[tid][k] = om[k];
      }
      if (tid == 0 && total > d.outlier_cap && a.overflow) atomicOr(a.overflow, TQK_OVF_OUTLIERS);
    } else if (tid < TQK_NOB) {
      a.p.ocount[obase * TQK_NOB + tid] = 0;
    }
    __syncthreads();

    // ---- codes: thread = (channel pair jp, token slice = wave); the slice's
    // rows belong to this wave alone, so a row's code bytes replace its first
    // D / 2 bytes right after the wave has read it.  A stored outlier takes the
    // grid level whose value is gmean -- NF4's zero level (code 7), or code 0
    // of a uniform grid -- so the dense part of a decode contributes gmean
    // there and the side-list adds val - gmean; export restores the
    // reference's code.
    for (int jp = lane; jp < D / 2; jp += 64) {
      const int kb = d.key_bits;
      const int per_q = (G + kEncWaves - 1) / kEncWaves;
      const int s0 = wv * per_q, s1 = min(G, s0 + per_q);
      const uint32_t zc = d.key_grid == 1 ? 0u : 7u;
      const float st00 = stat_s[2 * jp][0], st01 = stat_s[2 * jp][1];
      const float st10 = stat_s[2 * jp + 1][0], st11 = stat_s[2 * jp + 1][1];
      if (d.key_grid == 1) {
        // uniform: clip(round_half_even((x - min) / scale), 0, 2^bits - 1)
        const float qmax = (float)((1 << kb) - 1);
        for (int s = s0; s < s1; ++s) {
          const uint32_t xx = *reinterpret_cast<const uint32_t*>(&kt_s[s][2 * jp]);
          const float r0 = __builtin_rintf(__fdiv_rn(__fsub_rn(h2f((uint16_t)xx), st00), st01));
          const float r1 = __builtin_rintf(__fdiv_rn(__fsub_rn(h2f((uint16_t)(xx >> 16)), st10), st11));
          uint32_t b0 = (uint32_t)fminf(fmaxf(r0, 0.0f), qmax);
          uint32_t b1 = (uint32_t)fminf(fmaxf(r1, 0.0f), qmax);
          if (kout > 0) {
            const uint32_t om = omask_s[s][jp >> 4] >> (2 * (jp & 15));
            if (om & 1u) b0 = zc;
            if (om & 2u) b1 = zc;
          }
          // one table index per channel pair (the key row layout of tqk_common.h)
          kc_row(s)[jp] = (uint8_t)(kb == 4 ? ((rev4(b0) << 4) | rev4(b1)) : (b0 | (b1 << kb)));
        }
      } else {
        // asym-NF4 levels cent_l = mean + amax * NF4[l]
        float c0[16], c1[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) {
          c0[l] = __fadd_rn(st00, __fmul_rn(st01, kNF4[l]));
          c1[l] = __fadd_rn(st10, __fmul_rn(st11, kNF4[l]));
        }
        // With finite levels and a finite x no distance is NaN, and the
        // argmin needs only the strict comparison.  Sorted levels far enough
        // apart make it a count: for x >= c_l the distances x - c_l fall
        // strictly with l (their real gaps exceed the rounding, see below)
        // and for c_l > x they never fall, so the first argmin is the number
        // of strict decreases d_l < d_(l-1).  Every token of the group has
        // |x - mean| <= amax, so a distance is below R = 2 (|mean| + amax);
        // gaps of at least R * 2^-19 (16 ulps of R) cannot round away.
        bool lv_finite = true, spread = true;
#pragma unroll
        for (int l = 0; l < 16; ++l) lv_finite &= __builtin_isfinite(c0[l]) && __builtin_isfinite(c1[l]);
        {
          const float r0 = __fmul_rn(__fadd_rn(fabsf(st00), st01), 0x1p-18f);
          const float r1 = __fmul_rn(__fadd_rn(fabsf(st10), st11), 0x1p-18f);
#pragma unroll
          for (int l = 1; l < 16; ++l)
            spread &= __fsub_rn(c0[l], c0[l - 1]) >= r0 && __fsub_rn(c1[l], c1[l - 1]) >= r1;
          spread &= lv_finite;
        }
        for (int s = s0; s < s1; ++s) {
          const uint32_t xx = *reinterpret_cast<const uint32_t*>(&kt_s[s][2 * jp]);
          const float x0 = h2f((uint16_t)xx), x1 = h2f((uint16_t)(xx >> 16));
          uint32_t b0 = 0, b1 = 0;
          float d0 = fabsf(__fsub_rn(x0, c0[0])), d1 = fabsf(__fsub_rn(x1, c1[0]));
          const bool fin = lv_finite && (xx & 0x7C00u) != 0x7C00u && (xx & 0x7C000000u) != 0x7C000000u;
          if (__all(fin && spread)) {
#pragma unroll
            for (int l = 1; l < 16; ++l) {
              const float e0 = fabsf(__fsub_rn(x0, c0[l])), e1 = fabsf(__fsub_rn(x1, c1[l]));
              b0 += (e0 < d0) ? 1u : 0u;
              b1 += (e1 < d1) ? 1u : 0u;
              d0 = e0;
              d1 = e1;
            }
          } else if (__all(fin)) {
#pragma unroll
            for (int l = 1; l < 16; ++l) {
              const float e0 = fabsf(__fsub_rn(x0, c0[l])), e1 = fabsf(__fsub_rn(x1, c1[l]));
              if (e0 < d0) { d0 = e0; b0 = l; }
              if (e1 < d1) { d1 = e1; b1 = l; }
            }
          } else {
#pragma unroll
            for (int l = 1; l < 16; ++l) {
              const float e0 = fabsf(__fsub_rn(x0, c0[l])), e1 = fabsf(__fsub_rn(x1, c1[l]));
              // np.argmin: strictly smaller wins; the first NaN wins over any number
              if (e0 < d0 || (e0 != e0 && d0 == d0)) { d0 = e0; b0 = l; }
              if (e1 < d1 || (e1 != e1 && d1 == d1)) { d1 = e1; b1 = l; }
            }
          }
          if (kout > 0) {
            const uint32_t om = omask_s[s][jp >> 4] >> (2 * (jp & 15));
            if (om & 1u) b0 = zc;
            if (om & 2u) b1 = zc;
          }
          kc_row(s)[jp] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
        }
      }
    }
  }

  // ---- values -------------------------------------------------------------
  constexpr int VROW = D * VB / 8;
  const bool tiled = v_tiled(G, P, D, d.input_f32);
  // PolarQuant codes of the group's tokens (the value encode; PolarQuant keys
  // run it on the keys): norms to nout, codes staged in vc_s[token][channel]
  // (the first TQK_MAX_G * D bytes of the key tile area)
  auto polar_phase = [&](const void* ring, const void* chunk, float* nout, bool vcheck) {
    // Rotation: in pass p, wave w owns the 16 rotated channels [64p + 16w,
    // +16), lane l column e = 64p + 16w + (l & 15) of Pi_T (pi[e][0..D)) in
    // registers; the tokens' normalised rows sit in LDS (kVBatch at a time,
    // after the code staging area) and reach the lanes by DPP row broadcasts
    // (rotate_codes) -- no LDS broadcast reads, which would cost the LDS a
    // full wave's bandwidth each.
    float bnd[15];
#pragma unroll
    for (int k = 0; k < (1 << VB) - 1; ++k) bnd[k] = a.p.vbnd[k];
    constexpr int kVBatch = 64;  // rows per batch (rotate_codes takes at most 64)
    float (*u_s)[D] = reinterpret_cast<float (*)[D]>(&kt_s[0][0] + TQK_MAX_G * D / 2);
    for (int t0 = 0; t0 < G; t0 += kVBatch) {
      const int nb = min(kVBatch, G - t0);
      // (1) norms and normalised rows, four threads per token: thread q holds
      // channels 8m + 2q, 8m + 2q + 1 (pairwise_sumsq's partial sums)
      {
        const int tt = tid >> 2, q = tid & 3;
        if (tt < nb) {
          const int t = g * G + t0 + tt;
          const uint32_t* src = reinterpret_cast<const uint32_t*>(token_src<D>(a, ring, chunk, b, h, t));
          float x0[D / 8], x1[D / 8];
#pragma unroll
          for (int m = 0; m < D / 8; ++m) {
            const uint32_t w2 = src[4 * m + q];  // channels 8m + 2q, 8m + 2q + 1
            x0[m] = h2f((uint16_t)(w2 & 0xFFFFu));
            x1[m] = h2f((uint16_t)(w2 >> 16));
          }
          const float ss = pairwise_sumsq<D>(x0, x1, q);
          const float nrm = __builtin_sqrtf(ss);  // correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt)
          const float safe = fmaxf(nrm, 1e-30f);
#pragma unroll
          for (int m = 0; m < D / 8; ++m) {
            u_s[tt][8 * m + 2 * q] = __fdiv_rn(x0[m], safe);
            u_s[tt][8 * m + 2 * q + 1] = __fdiv_rn(x1[m], safe);
          }
          if (q == 0) {
            nout[page_row(a.p.block_table, d.max_pages_per_seq, b, t, P, d.n_pages, h)] = nrm;
            if (vcheck && nrm > TQK_MAX_VNORM && a.overflow) atomicOr(a.overflow, TQK_OVF_VNORM);
          }
        }
      }
      __syncthreads();
      // (2) rotation and codes, D / (16 * kEncWaves) passes over the channels
      for (int pass = 0; pass < D / (16 * kEncWaves); ++pass)
        rotate_codes<D, VB>(a.p.pi, u_s, nb, 16 * kEncWaves * pass + 16 * wv + (lane & 15), lane, bnd,
                            vc_s + t0);
      __syncthreads();
    }
  };
  // code row of token t for the key write-out
  const uint8_t* kc_base = kc_row(0);
  int kc_stride = (D + 8) * 2;
  if (d.key_grid == 2) {
    // PolarQuant keys (turboquant_pro/core.py:542-617 with kind="key"): the
    // value encode on the key tokens, norms to knorm, then each row's codes
    // turned in place (one wave per row) into one table index per channel
    // pair; the per-channel stats are the identity (scale 1, mean 0) and
    // there is no side-list
    polar_phase(a.p.hot_k, a.chunk_k, a.p.knorm, false);
    for (int t = wv; t < G; t += kEncWaves) {
      // every pair of the row read before any index is written over it
      constexpr int NPL = (D / 2 + 63) / 64;  // channel pairs per lane
      uint32_t f[NPL];
#pragma unroll
      for (int k = 0; k < NPL; ++k) {
        const int pr = lane + 64 * k;
        const uint32_t cc = pr < D / 2 ? *reinterpret_cast<const uint16_t*>(&vc_s[t][2 * pr]) : 0u;
        const uint32_t c0 = cc & 0xFFu, c1 = cc >> 8;
        f[k] = d.key_bits == 4 ? ((rev4(c0) << 4) | rev4(c1)) : (c0 | (c1 << d.key_bits));
      }
#pragma unroll
      for (int k = 0; k < NPL; ++k)
        if (lane + 64 * k < D / 2) vc_s[t][lane + 64 * k] = (uint8_t)f[k];
    }
    kc_base = &vc_s[0][0];
    kc_stride = D;
    if (tid < D) {
      a.p.gscale[mbase + tid] = 1.0f;
      a.p.gmean[mbase + tid] = 0.0f;
    }
    if (tid < TQK_NOB) a.p.ocount[obase * TQK_NOB + tid] = 0;
  }
  __syncthreads();
  // key code rows, one 32-channel chunk (16 pair indices) per thread
  const int KROW = k_row_bytes(d.key_bits, D);
  for (int idx = tid; idx < G * (D / 32); idx += kEncThreads) {
    const int t = idx / (D / 32), ch = idx % (D / 32);
    const size_t row = page_row(a.p.block_table, d.max_pages_per_seq, b, g * G + t, P, d.n_pages, h);
    const uint4 f16 = *reinterpret_cast<const uint4*>(kc_base + (size_t)t * kc_stride + 16 * ch);
    if (d.key_bits == 4) {
      *reinterpret_cast<uint4*>(a.p.kcodes + row * KROW + 16 * ch) = f16;
    } else {
      // 16 fields of 2*kb bits, little-endian, into kb dwords
      const int kb = d.key_bits;
      const uint32_t fw[4] = {f16.x, f16.y, f16.z, f16.w};
      uint32_t o[3] = {0u, 0u, 0u};
      for (int i = 0; i < 16; ++i) {
        const uint32_t f = (fw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        const int bo = 2 * kb * i, w = bo >> 5, sh = bo & 31;
        o[w] |= f << sh;
        if (sh + 2 * kb > 32) o[w + 1] |= f >> (32 - sh);
      }
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.p.kcodes + row * KROW + 4 * kb * ch);
      for (int w = 0; w < kb; ++w) dst[w] = o[w];
    }
  }
  __syncthreads();
  polar_phase(a.p.hot_v, a.chunk_v, a.p.vnorm, true);
  // (3) the code rows: 4-token x 8-channel units of 16-token tiles, or the
  // reference's little-endian bit stream per token
  if (D == TQK_D && tiled) {
    // one unit = tokens [16T + 4lg, +4) x channels [8c, +8) of 16-token tile T
    for (int un = tid; un < (G / 16) * 64; un += kEncThreads) {
      const int T = un >> 6, lg = (un >> 4) & 3, c = un & 15;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const uint32_t code = vc_s[16 * T + 4 * lg + uu][8 * c + nt];
          const int bit = v_unit_bit(uu, nt, VB);
          w[bit >> 5] |= code << (bit & 31);
          if ((bit & 31) + VB > 32) w[(bit >> 5) + 1] |= code >> (32 - (bit & 31));
        }
      }
      const int t0 = g * G + 16 * T;  // tile start (absolute token), never straddles a page
      const size_t row0 = page_row(a.p.block_table, d.max_pages_per_seq, b, t0, P, d.n_pages, h);
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.p.vcodes + row0 * VROW + v_unit_offset(lg, c, VROW));
#pragma unroll
      for (int k = 0; k < VROW / 16; ++k) dst[k] = w[k];
    }
  } else if (tid < G) {
    uint32_t outw[VROW / 4];
#pragma unroll
    for (int k = 0; k < VROW / 4; ++k) outw[k] = 0u;
#pragma unroll
    for (int e = 0; e < D; ++e) {
      const uint32_t code = vc_s[tid][e];
      const int bitpos = e * VB;  // little-endian bit stream (3-bit: 8 codes per 24 bits)
      outw[bitpos >> 5] |= code << (bitpos & 31);
      if ((bitpos & 31) + VB > 32) outw[(bitpos >> 5) + 1] |= code >> (32 - (bitpos & 31));
    }
    const size_t row = page_row(a.p.block_table, d.max_pages_per_seq, b, g * G + tid, P, d.n_pages, h);
    // 16-byte stores where the row is whole 16-byte pieces (3-bit rows at
    // head_dim 64 are 24 bytes: dword stores)
    if constexpr (VROW % 16 == 0) {
      uint4* dst = reinterpret_cast<uint4*>(a.p.vcodes + row * VROW);
#pragma unroll
      for (int k = 0; k < VROW / 16; ++k)
        dst[k] = make_uint4(outw[4 * k], outw[4 * k + 1], outw[4 * k + 2], outw[4 * k + 3]);
    } else {
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.p.vcodes + row * VROW);
#pragma unroll
      for (int k = 0; k < VROW / 4; ++k) dst[k] = outw[k];
    }
  }
}


// ---------------------------------------------------------------------------
// Quantize-on-flush of an fp32 cache (input_f32): the same codes, stats and
// side-list as the fp16 encode, in the same NumPy operation order, from fp32
// rows read through L1/L2 (an fp32 group does not fit the LDS key tile).  The
// side-list positions keep the reference's codes (argmin on the fp32 value);
// value codes are per-token rows.  Value norms are not bounded: the VALU
// decode, the one that serves fp32 caches, keeps its weights in fp32.
template <int VB, int D>
__global__ __launch_bounds__(kEncThreads) void tqk_encode_group_f32(EncodeArgs a) {
  const int item = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const tqk_cache_desc& d = a.d;
  const int b = a.items[2 * item], g = a.items[2 * item + 1];
  const int G = d.group_tokens, P = d.page_tokens, Hkv = d.n_kv_heads;
  const int slot = a.p.group_table[(size_t)b * d.max_groups_per_seq + g];
  const int kout = d.outliers_per_channel;
  const size_t mbase = ((size_t)slot * Hkv + h) * D;
  const size_t obase = (size_t)slot * Hkv + h;
  constexpr int kVBatch = 64;  // rows per value batch (rotate_codes takes at most 64)
  constexpr int VROW = D * VB / 8;

  __shared__ const float* krow_s[TQK_MAX_G];                // source row of each key token
  __shared__ float stat_s[D][2];                             // (mean, amax) or (min, scale)
  __shared__ float thr_s[D];                                 // outlier magnitude threshold
  __shared__ __align__(16) uint8_t kc_s[TQK_MAX_G][D / 2];   // table index per (token, channel pair)
  __shared__ __align__(16) float u_s[kVBatch][D];
  __shared__ __align__(16) uint8_t vc_s[kVBatch][D];
  __shared__ int32_t wsum_s[kEncWaves];

  for (int t = tid; t < G; t += kEncThreads)
    krow_s[t] = token_src<D, float>(a, a.p.hot_k, a.chunk_k, b, h, g * G + t);
  __syncthreads();

  // norms and normalised rows of tokens [t0, t0 + nb) (four threads per
  // token, pairwise_sumsq), then their rotated codes into vc_s
  float bnd[15];
#pragma unroll
  for (int k = 0; k < (1 << VB) - 1; ++k) bnd[k] = a.p.vbnd[k];
  auto polar_batch = [&](const void* ring, const void* chunk, int t0, int nb, float* nout) {
    const int tt = tid >> 2, q = tid & 3;
    if (tt < nb) {
      const int t = g * G + t0 + tt;
      const float2* src = reinterpret_cast<const float2*>(token_src<D, float>(a, ring, chunk, b, h, t));
      float x0[D / 8], x1[D / 8];
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        const float2 w2 = src[4 * m + q];  // channels 8m + 2q, 8m + 2q + 1
        x0[m] = w2.x;
        x1[m] = w2.y;
      }
      const float nrm = __builtin_sqrtf(pairwise_sumsq<D>(x0, x1, q));
      const float safe = fmaxf(nrm, 1e-30f);
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        u_s[tt][8 * m + 2 * q] = __fdiv_rn(x0[m], safe);
        u_s[tt][8 * m + 2 * q + 1] = __fdiv_rn(x1[m], safe);
      }
      if (q == 0) nout[page_row(a.p.block_table, d.max_pages_per_seq, b, t, P, d.n_pages, h)] = nrm;
    }
    __syncthreads();
    for (int pass = 0; pass < D / (16 * kEncWaves); ++pass)
      rotate_codes<D, VB>(a.p.pi, u_s, nb, 16 * kEncWaves * pass + 16 * wv + (lane & 15), lane, bnd, vc_s);
    __syncthreads();
  };

  if (d.key_grid != 2) {
    auto X = [&](int s, int j) { return krow_s[s][j]; };
    // ---- per-channel statistics, thread j: channel j
    if (tid < D) {
      const int j = tid;
      float st0, st1;
      if (d.key_grid == 1) {
        float mn = X(0, j), mx = mn;
        bool nan = (mn != mn);
        for (int s = 1; s < G; ++s) {
          const float xv = X(s, j);
          nan |= (xv != xv);
          mn = fminf(mn, xv);
          mx = fmaxf(mx, xv);
        }
        st1 = nan ? __builtin_nanf("") : __fdiv_rn(fmaxf(__fsub_rn(mx, mn), 1e-8f), (float)((1 << d.key_bits) - 1));
        st0 = nan ? __builtin_nanf("") : mn;
      } else {
        float mu;
        if (d.zero_point == 2) {
          mu = a.p.zp_mean[((size_t)g * Hkv + h) * D + j];
        } else {
          float acc = 0.0f;
          for (int s = 0; s < G; ++s) acc = __fadd_rn(acc, X(s, j));
          mu = (float)((double)acc / (double)G);
          if (d.zero_point == 1) mu = __fmul_rn(mu, ((d.dc_mask[j >> 5] >> (j & 31)) & 1u) ? 1.0f : 0.0f);
        }
        float amax = 0.0f;
        bool nan = (mu != mu);
        for (int s = 0; s < G; ++s) {
          const float dv = fabsf(__fsub_rn(X(s, j), mu));
          nan |= (dv != dv);
          amax = fmaxf(amax, dv);
        }
        st0 = mu;
        st1 = nan ? __builtin_nanf("") : fmaxf(amax, 1e-8f);
      }
      stat_s[j][0] = st0;
      stat_s[j][1] = st1;
      a.p.gscale[mbase + j] = st1;
      a.p.gmean[mbase + j] = st0;
      // outlier threshold: the k-th largest |x| of the channel as the largest
      // fp32 magnitude pattern T with #{ |x_s| >= T } >= k (NaN patterns order
      // above inf, as np.partition places NaN last); the k <= 8 largest are
      // kept directly, otherwise a bitwise search
      if (kout > 0 && kout < G) {
        uint32_t T = 0;
        if (kout <= 8) {
          uint32_t top[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) top[i] = 0u;
          for (int s = 0; s < G; ++s) {
            uint32_t v = __float_as_uint(fabsf(X(s, j)));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const uint32_t hi = max(top[i], v);
              v = min(top[i], v);
              top[i] = hi;
            }
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i == kout - 1) T = top[i];
        } else {
          for (int bit = 30; bit >= 0; --bit) {
            const uint32_t cand = T | (1u << bit);
            int cnt = 0;
            for (int s = 0; s < G; ++s) cnt += __float_as_uint(fabsf(X(s, j))) >= cand ? 1 : 0;
            if (cnt >= kout) T = cand;
          }
        }
        thr_s[j] = __uint_as_float(T);  // a NaN threshold selects nothing, as |x| >= NaN
      }
    }
    __syncthreads();

    // ---- outlier side-list in flat (token, channel) order, one token per
    // thread (the cumulative counts at every TQK_OBLK-token boundary as the
    // fp16 encode writes them)
    if (kout > 0) {
      const bool all = kout >= G;
      int cnt = 0;
      if (tid < G) {
        const float* row = krow_s[tid];
        for (int j = 0; j < D; ++j) cnt += (all || fabsf(row[j]) >= thr_s[j]) ? 1 : 0;
      }
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      if (lane == 63) wsum_s[wv] = incl;
      __syncthreads();
      int wofs = 0, total = 0;
      for (int w = 0; w < kEncWaves; ++w) {
        if (w < wv) wofs += wsum_s[w];
        total += wsum_s[w];
      }
      int off = wofs + incl - cnt;
      if (tid < G && ((tid + 1) % TQK_OBLK) == 0 && (tid + 1) / TQK_OBLK <= TQK_NOB)
        a.p.ocount[obase * TQK_NOB + (tid + 1) / TQK_OBLK - 1] = off + cnt;
      if (tid < TQK_NOB && TQK_OBLK * (tid + 1) > G) a.p.ocount[obase * TQK_NOB + tid] = total;
      if (tid < G && cnt > 0) {
        const float* row = krow_s[tid];
        for (int j = 0; j < D && off < d.outlier_cap; ++j) {
          const float xv = row[j];
          if (all || fabsf(xv) >= thr_s[j]) {
            a.p.oent[obase * d.outlier_cap + off] = (uint32_t)(tid * D + j) | ((uint32_t)f2h(xv) << 16);
            ++off;
          }
        }
      }
      if (tid == 0 && total > d.outlier_cap && a.overflow) atomicOr(a.overflow, TQK_OVF_OUTLIERS);
    } else if (tid < TQK_NOB) {
      a.p.ocount[obase * TQK_NOB + tid] = 0;
    }

    // ---- codes: thread = (channel pair, token slice = wave), the reference's
    // code everywhere (side-list positions included)
    const int kb = d.key_bits;
    const int per_q = (G + kEncWaves - 1) / kEncWaves;
    const int s0 = wv * per_q, s1 = min(G, s0 + per_q);
    for (int jp = lane; jp < D / 2; jp += 64) {
      const float st00 = stat_s[2 * jp][0], st01 = stat_s[2 * jp][1];
      const float st10 = stat_s[2 * jp + 1][0], st11 = stat_s[2 * jp + 1][1];
      if (d.key_grid == 1) {
        const float qmax = (float)((1 << kb) - 1);
        for (int s = s0; s < s1; ++s) {
          const float2 xx = *reinterpret_cast<const float2*>(krow_s[s] + 2 * jp);
          const float r0 = __builtin_rintf(__fdiv_rn(__fsub_rn(xx.x, st00), st01));
          const float r1 = __builtin_rintf(__fdiv_rn(__fsub_rn(xx.y, st10), st11));
          const uint32_t b0 = (uint32_t)fminf(fmaxf(r0, 0.0f), qmax);
          const uint32_t b1 = (uint32_t)fminf(fmaxf(r1, 0.0f), qmax);
          kc_s[s][jp] = (uint8_t)(kb == 4 ? ((rev4(b0) << 4) | rev4(b1)) : (b0 | (b1 << kb)));
        }
      } else {
        float c0[16], c1[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) {
          c0[l] = __fadd_rn(st00, __fmul_rn(st01, kNF4[l]));
          c1[l] = __fadd_rn(st10, __fmul_rn(st11, kNF4[l]));
        }
        for (int s = s0; s < s1; ++s) {
          const float2 xx = *reinterpret_cast<const float2*>(krow_s[s] + 2 * jp);
          uint32_t b0 = 0, b1 = 0;
          float d0 = fabsf(__fsub_rn(xx.x, c0[0])), d1 = fabsf(__fsub_rn(xx.y, c1[0]));
#pragma unroll
          for (int l = 1; l < 16; ++l) {
            const float e0 = fabsf(__fsub_rn(xx.x, c0[l])), e1 = fabsf(__fsub_rn(xx.y, c1[l]));
            // np.argmin: strictly smaller wins; the first NaN wins over any number
            if (e0 < d0 || (e0 != e0 && d0 == d0)) { d0 = e0; b0 = l; }
            if (e1 < d1 || (e1 != e1 && d1 == d1)) { d1 = e1; b1 = l; }
          }
          kc_s[s][jp] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
        }
      }
    }
  } else {
    // PolarQuant keys: the value encode on the key tokens, norms to knorm;
    // each token's codes become one table index per channel pair
    for (int t0 = 0; t0 < G; t0 += kVBatch) {
      const int nb = min(kVBatch, G - t0);
      polar_batch(a.p.hot_k, a.chunk_k, t0, nb, a.p.knorm);
      for (int i = tid; i < nb * (D / 2); i += kEncThreads) {
        const int t = i / (D / 2), pr = i % (D / 2);
        const uint32_t c0 = vc_s[t][2 * pr], c1 = vc_s[t][2 * pr + 1];
        kc_s[t0 + t][pr] = (uint8_t)(d.key_bits == 4 ? ((rev4(c0) << 4) | rev4(c1)) : (c0 | (c1 << d.key_bits)));
      }
    }
    if (tid < D) {
      a.p.gscale[mbase + tid] = 1.0f;
      a.p.gmean[mbase + tid] = 0.0f;
    }
    if (tid < TQK_NOB) a.p.ocount[obase * TQK_NOB + tid] = 0;
  }
  __syncthreads();
  // key code rows, one 32-channel chunk (16 table indices) per thread
  const int KROW = k_row_bytes(d.key_bits, D);
  for (int idx = tid; idx < G * (D / 32); idx += kEncThreads) {
    const int t = idx / (D / 32), ch = idx % (D / 32);
    const size_t row = page_row(a.p.block_table, d.max_pages_per_seq, b, g * G + t, P, d.n_pages, h);
    const uint4 f16 = *reinterpret_cast<const uint4*>(&kc_s[t][16 * ch]);
    if (d.key_bits == 4) {
      *reinterpret_cast<uint4*>(a.p.kcodes + row * KROW + 16 * ch) = f16;
    } else {
      const int kb = d.key_bits;
      const uint32_t fw[4] = {f16.x, f16.y, f16.z, f16.w};
      uint32_t o[3] = {0u, 0u, 0u};
      for (int i = 0; i < 16; ++i) {
        const uint32_t f = (fw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        const int bo = 2 * kb * i, w = bo >> 5, sh = bo & 31;
        o[w] |= f << sh;
        if (sh + 2 * kb > 32) o[w + 1] |= f >> (32 - sh);
      }
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.p.kcodes + row * KROW + 4 * kb * ch);
      for (int w = 0; w < kb; ++w) dst[w] = o[w];
    }
  }
  // ---- values, kVBatch tokens at a time: codes, then the reference's
  // little-endian bit stream per token
  for (int t0 = 0; t0 < G; t0 += kVBatch) {
    const int nb = min(kVBatch, G - t0);
    polar_batch(a.p.hot_v, a.chunk_v, t0, nb, a.p.vnorm);
    if (tid < nb) {
      uint32_t outw[VROW / 4];
#pragma unroll
      for (int k = 0; k < VROW / 4; ++k) outw[k] = 0u;
#pragma unroll
      for (int e = 0; e < D; ++e) {
        const uint32_t code = vc_s[tid][e];
        const int bitpos = e * VB;
        outw[bitpos >> 5] |= code << (bitpos & 31);
        if ((bitpos & 31) + VB > 32) outw[(bitpos >> 5) + 1] |= code >> (32 - (bitpos & 31));
      }
      const size_t row = page_row(a.p.block_table, d.max_pages_per_seq, b, g * G + t0 + tid, P, d.n_pages, h);
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.p.vcodes + row * VROW);
#pragma unroll
      for (int k = 0; k < VROW / 4; ++k) dst[k] = outw[k];
    }
    __syncthreads();  // vc_s is the next batch's
  }
}


struct HotArgs {
  tqk_cache_desc d;
  uint8_t* hot_k;
  uint8_t* hot_v;
  const int32_t* prev_len;
  const int32_t* n_new;
  const int32_t* hot_start;
  const uint8_t* chunk_k;
  const uint8_t* chunk_v;
  int chunk_tokens;
};

constexpr int kHotSlice = 64;  // tokens per workgroup of the ring copy

// grid (batch, Hkv, slices): copies the surviving new tokens into the ring,
// kHotSlice tokens per workgroup and round (slices stride by gridDim.z), so a
// chunk's copy spreads over the whole chip instead of one workgroup per
// (sequence, kv head).
__global__ __launch_bounds__(kThreads) void tqk_append_hot_kernel(HotArgs a) {
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const tqk_cache_desc& d = a.d;
  const int prev = a.prev_len[b], nn = a.n_new[b];
  const int t0 = max(prev, a.hot_start[b]), t1 = prev + nn;
  const int R = d.hot_ring;
  const size_t rb = ((size_t)b * d.n_kv_heads + h) * R;
  const size_t cb = ((size_t)b * d.n_kv_heads + h) * a.chunk_tokens;
  const int rowb = d.head_dim * (d.input_f32 ? 4 : 2), nc = rowb / 16;  // 16-byte pieces per row
  for (int s0 = t0 + (int)blockIdx.z * kHotSlice; s0 < t1; s0 += (int)gridDim.z * kHotSlice) {
    const int n = min(kHotSlice, t1 - s0);
    for (int idx = tid; idx < n * nc; idx += kThreads) {
      const int t = s0 + idx / nc, c = idx % nc;
      const size_t src = (cb + (t - prev)) * rowb;
      const size_t dst = (rb + (t % R)) * rowb;
      reinterpret_cast<uint4*>(a.hot_k + dst)[c] = reinterpret_cast<const uint4*>(a.chunk_k + src)[c];
      reinterpret_cast<uint4*>(a.hot_v + dst)[c] = reinterpret_cast<const uint4*>(a.chunk_v + src)[c];
    }
  }
}

struct DequantArgs {
  tqk_cache_desc d;
  tqk_cache_ptrs p;
  const int32_t* items;
  float* kout;
  float* vout;
};

// grid (n_items, Hkv), one token per thread: reconstruct keys (grid value then
// the fp16 outlier overwrite) and values ((cent[code] @ Pi) * norm, NumPy order).
template <int VB, int D>
__global__ __launch_bounds__(kThreads) void tqk_dequant_group(DequantArgs a) {
  constexpr int VROW = D * VB / 8;
  const int item = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const tqk_cache_desc& d = a.d;
  const int b = a.items[2 * item], g = a.items[2 * item + 1];
  const int G = d.group_tokens, P = d.page_tokens, Hkv = d.n_kv_heads;
  const int slot = a.p.group_table[(size_t)b * d.max_groups_per_seq + g];
  const size_t mbase = ((size_t)slot * Hkv + h) * D;
  float* ko = a.kout + ((size_t)item * Hkv + h) * G * D;
  float* vo = a.vout + ((size_t)item * Hkv + h) * G * D;
  if (tid < G) {
    const size_t row = page_row(a.p.block_table, d.max_pages_per_seq, b, g * G + tid, P, d.n_pages, h);
    const int kb = d.key_bits, KROW = k_row_bytes(kb, D);
    uint32_t rw[D / 8];
    const uint32_t* kr = reinterpret_cast<const uint32_t*>(a.p.kcodes + row * KROW);
    for (int w = 0; w < KROW / 4; ++w) rw[w] = kr[w];
    if (d.key_grid == 2) {
      // PolarQuant keys: (cent[code] @ Pi) * norm, as the values below
      float yk[D];
      for (int jj = 0; jj < D / 2; ++jj) {
        const uint32_t f = k_pair_index(rw, kb, jj);
        yk[2 * jj] = a.p.vcent[k_code_even(f, kb)];
        yk[2 * jj + 1] = a.p.vcent[k_code_odd(f, kb)];
      }
      const float kn = a.p.knorm[row];
      for (int e = 0; e < D; ++e) {
        float x = 0.f;
#pragma unroll
        for (int j = 0; j < D; ++j) x = __fadd_rn(x, __fmul_rn(yk[j], a.p.pi[j * D + e]));
        ko[(size_t)tid * D + e] = __fmul_rn(x, kn);
      }
    } else {
      for (int jj = 0; jj < D / 2; ++jj) {
        const uint32_t f = k_pair_index(rw, kb, jj);
        const int j0 = 2 * jj, j1 = 2 * jj + 1;
        ko[(size_t)tid * D + j0] =
            __fadd_rn(__fmul_rn(a.p.gscale[mbase + j0], key_level(d.key_grid, k_code_even(f, kb))), a.p.gmean[mbase + j0]);
        ko[(size_t)tid * D + j1] =
            __fadd_rn(__fmul_rn(a.p.gscale[mbase + j1], key_level(d.key_grid, k_code_odd(f, kb))), a.p.gmean[mbase + j1]);
      }
    }
    float y[D];
    if (D == TQK_D && v_tiled(G, P, D, d.input_f32)) {
      // unit (lg, c) of the token's 16-token tile; tile rows start at row - (t % 16)
      const int tt = (g * G + tid) % 16;
      const uint8_t* tile = a.p.vcodes + (row - tt) * VROW;
      const int lg = tt >> 2, uu = tt & 3;
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const uint8_t* un = tile + v_unit_offset(lg, j >> 3, VROW);
        const int bit = v_unit_bit(uu, j & 7, VB);
        const uint32_t w = un[bit >> 3] | ((uint32_t)un[min((bit >> 3) + 1, VROW / 4 - 1)] << 8);
        y[j] = a.p.vcent[(w >> (bit & 7)) & ((1u << VB) - 1)];
      }
    } else {
      const uint8_t* vr = a.p.vcodes + row * VROW;
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const int bitpos = j * VB;
        uint32_t w = vr[bitpos >> 3] | ((uint32_t)vr[min((bitpos >> 3) + 1, VROW - 1)] << 8);
        y[j] = a.p.vcent[(w >> (bitpos & 7)) & ((1u << VB) - 1)];
      }
    }
    const float nrm = a.p.vnorm[row];
    for (int e = 0; e < D; ++e) {
      float x = 0.f;
#pragma unroll
      for (int j = 0; j < D; ++j) x = __fadd_rn(x, __fmul_rn(y[j], a.p.pi[j * D + e]));
      vo[(size_t)tid * D + e] = __fmul_rn(x, nrm);
    }
  }
  __syncthreads();
  const size_t obase = (size_t)slot * Hkv + h;
  const int no = min(a.p.ocount[obase * TQK_NOB + TQK_NOB - 1], d.outlier_cap);
  for (int e = tid; e < no; e += kThreads) {
    const uint32_t ent = a.p.oent[obase * d.outlier_cap + e];
    ko[ent & 0xFFFFu] = h2f((uint16_t)(ent >> 16));
  }
}

// one kernel instance per (value bits, head_dim)
template <int D>
void launch_by_vb(int vb, dim3 grid, hipStream_t st, const EncodeArgs& a) {
  if (a.d.input_f32) {
    if (vb == 2)
      hipLaunchKernelGGL((tqk_encode_group_f32<2, D>), grid, dim3(kEncThreads), 0, st, a);
    else if (vb == 3)
      hipLaunchKernelGGL((tqk_encode_group_f32<3, D>), grid, dim3(kEncThreads), 0, st, a);
    else
      hipLaunchKernelGGL((tqk_encode_group_f32<4, D>), grid, dim3(kEncThreads), 0, st, a);
  } else if (vb == 2) {
    hipLaunchKernelGGL((tqk_encode_group<2, D>), grid, dim3(kEncThreads), 0, st, a);
  } else if (vb == 3) {
    hipLaunchKernelGGL((tqk_encode_group<3, D>), grid, dim3(kEncThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL((tqk_encode_group<4, D>), grid, dim3(kEncThreads), 0, st, a);
  }
}
template <int D>
void launch_by_vb(int vb, dim3 grid, hipStream_t st, const DequantArgs& a) {
  if (vb == 2)
    hipLaunchKernelGGL((tqk_dequant_group<2, D>), grid, dim3(kThreads), 0, st, a);
  else if (vb == 3)
    hipLaunchKernelGGL((tqk_dequant_group<3, D>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((tqk_dequant_group<4, D>), grid, dim3(kThreads), 0, st, a);
}

}  // namespace

extern "C" {

int tqk_encode_groups(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                      int32_t n_items, const int32_t* items, const int32_t* prev_len,
                      const void* chunk_k, const void* chunk_v, int32_t chunk_tokens,
                      int32_t* overflow, void* stream) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || batch <= 0 || n_items < 0 || chunk_tokens < 0) return TQK_EINVAL;
  if (n_items == 0) return TQK_OK;
  if (!items || !prev_len) return TQK_EINVAL;
  EncodeArgs a;
  a.d = *d;
  a.p = *p;
  a.items = items;
  a.prev_len = prev_len;
  a.chunk_k = chunk_k;
  a.chunk_v = chunk_v;
  a.chunk_tokens = chunk_tokens;
  a.overflow = overflow;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (d->key_grid == 0 && d->zero_point == 2 && !p->zp_mean) return TQK_EINVAL;
  if (d->key_grid == 2 && !p->knorm) return TQK_EINVAL;
  const dim3 grid(n_items, d->n_kv_heads);
  if (d->head_dim == 64)
    launch_by_vb<64>(d->value_bits, grid, st, a);
  else if (d->head_dim == 128)
    launch_by_vb<128>(d->value_bits, grid, st, a);
  else
    launch_by_vb<256>(d->value_bits, grid, st, a);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int tqk_append_hot(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                   const int32_t* prev_len, const int32_t* n_new, const int32_t* hot_start,
                   const void* chunk_k, const void* chunk_v, int32_t chunk_tokens,
                   void* stream) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || batch <= 0 || !prev_len || !n_new || !hot_start || !chunk_k || !chunk_v ||
      chunk_tokens <= 0)
    return TQK_EINVAL;
  HotArgs a;
  a.d = *d;
  a.hot_k = static_cast<uint8_t*>(p->hot_k);
  a.hot_v = static_cast<uint8_t*>(p->hot_v);
  a.prev_len = prev_len;
  a.n_new = n_new;
  a.hot_start = hot_start;
  a.chunk_k = static_cast<const uint8_t*>(chunk_k);
  a.chunk_v = static_cast<const uint8_t*>(chunk_v);
  a.chunk_tokens = chunk_tokens;
  // the surviving tokens of a sequence number at most min(chunk, ring)
  const int span = min(chunk_tokens, d->hot_ring);
  const int slices = max(1, (span + kHotSlice - 1) / kHotSlice);
  hipLaunchKernelGGL(tqk_append_hot_kernel, dim3(batch, d->n_kv_heads, slices), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int tqk_dequant_groups(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t n_items,
                       const int32_t* items, float* kout, float* vout, void* stream) {
  int rc = tqk_check_desc(d);
  if (rc != TQK_OK) return rc;
  if (!p || n_items < 0 || (n_items > 0 && (!items || !kout || !vout))) return TQK_EINVAL;
  if (n_items == 0) return TQK_OK;
  if (d->key_grid == 2 && !p->knorm) return TQK_EINVAL;
  DequantArgs a;
  a.d = *d;
  a.p = *p;
  a.items = items;
  a.kout = kout;
  a.vout = vout;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(n_items, d->n_kv_heads);
  if (d->head_dim == 64)
    launch_by_vb<64>(d->value_bits, grid, st, a);
  else if (d->head_dim == 128)
    launch_by_vb<128>(d->value_bits, grid, st, a);
  else
    launch_by_vb<256>(d->value_bits, grid, st, a);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

}  // extern "C"
