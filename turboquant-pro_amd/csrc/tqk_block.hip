// Stateless block quantizers and their reconstruction (gfx950).
//
// One (B, H, S, D) block per call, every (b, h) pair one quantization group of
// S tokens (any S >= 1), fp16 or fp32 input, outputs in the reference
// containers' layouts: the whole-layer records of the plugin / block-store
// path, which the cache's 256-token group encode does not cover.
//
// Bit-exactness contract (compiled with -ffp-contract=off, explicitly rounded
// __f*_rn operations), the same NumPy operation order as the group encode:
//   keys   (turboquant_pro/per_channel_kv.py:269-401)
//     asym-NF4: mu = token-order sequential fp32 sum / S (a float64 division,
//               then fp32), times the DC mask ("sparse") or given ("bias");
//               amax = max(max_s |x_s - mu|, 1e-8); cent = mu + amax * NF4[l];
//               code = first argmin_l |x - cent_l|
//     uniform:  scale = max(max - min, 1e-8) / (2^bits - 1);
//               code = clip(rint((x - min) / scale), 0, 2^bits - 1)
//   key packing (per_channel_kv.py:87-100): each code's bits LSB first, in
//   MSB-first bytes, codes in (b, h, s, j) order (4-bit: byte n =
//   rev4(code[2n]) << 4 | rev4(code[2n+1]); a token row is D * bits / 8 bytes)
//     outliers: threshold = k-th largest |x| over s; every |x| >= it, (s, j) order
//   values (turboquant_pro/core.py:569-606): pairwise norm, u = x / max(norm, 1e-30),
//     y_e = sequential over d of u_d * Pi[e][d], code = #{ boundaries < y_e }
#include "tqk_common.h"

namespace {

constexpr int kKbThreads = 256;  // key dequant kernels
constexpr int kVbThreads = 512;  // value block: 64 tokens per workgroup
constexpr int kVbTokens = 64;

__device__ __forceinline__ float load_x(const void* x, int f32, size_t i) {
  return f32 ? reinterpret_cast<const float*>(x)[i] : h2f(reinterpret_cast<const uint16_t*>(x)[i]);
}
// N values of x at i0, i0 + stride, ..., every load issued before any is used
template <int N>
__device__ __forceinline__ void load_xn(const void* x, int f32, size_t i0, size_t stride, float (&v)[N]) {
  if (f32) {
    const float* p = reinterpret_cast<const float*>(x) + i0;
#pragma unroll
    for (int u = 0; u < N; ++u) v[u] = p[u * stride];
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(x) + i0;
    uint16_t r[N];
#pragma unroll
    for (int u = 0; u < N; ++u) r[u] = p[u * stride];
#pragma unroll
    for (int u = 0; u < N; ++u) v[u] = h2f(r[u]);
  }
}
// f(s, x[s, col]) for s = s0, s0 + st, ... < s1, in that order, the loads of
// 32 tokens at a time in flight (rows of D elements; one or two waves per SIMD
// run these loops, so each batch waits one memory latency)
template <int D, typename F>
__device__ __forceinline__ void for_tokens(const void* x, int f32, size_t col, int s0, int s1, int st, F f) {
  constexpr int N = 32;
  int s = s0;
  for (; s + (N - 1) * st < s1; s += N * st) {
    float v[N];
    load_xn<N>(x, f32, col + (size_t)s * D, (size_t)st * D, v);
#pragma unroll
    for (int u = 0; u < N; ++u) f(s + u * st, v[u]);
  }
  for (; s < s1; s += st) f(s, load_x(x, f32, col + (size_t)s * D));
}
// f(s, x[s, col], x[s, col + 1]) in token order, 16 tokens' loads in flight
template <int D, typename F>
__device__ __forceinline__ void for_token_pairs(const void* x, int f32, size_t col, int s0, int s1, F f) {
  constexpr int N = 16;
  int s = s0;
  for (; s + N - 1 < s1; s += N) {
    float v0[N], v1[N];
    load_xn<N>(x, f32, col + (size_t)s * D, D, v0);
    load_xn<N>(x, f32, col + 1 + (size_t)s * D, D, v1);
#pragma unroll
    for (int u = 0; u < N; ++u) f(s + u, v0[u], v1[u]);
  }
  for (; s < s1; ++s) f(s, load_x(x, f32, col + (size_t)s * D), load_x(x, f32, col + 1 + (size_t)s * D));
}
__device__ __forceinline__ bool dc_channel(const tqk_block_desc& d, int j) {
  return (d.dc_mask[j >> 5] >> (j & 31)) & 1u;
}
// code c of channel j into a token row of little-endian dwords, in the
// reference's bit order (bit k of c at stream position j * bits + k, streams
// filling bytes from their most significant bit)
__device__ __forceinline__ void put_code_ref(uint32_t* rw, int j, int bits, uint32_t c) {
  for (int k = 0; k < bits; ++k) {
    const int p = j * bits + k;
    rw[p >> 5] |= ((c >> k) & 1u) << (8 * ((p >> 3) & 3) + 7 - (p & 7));
  }
}
// code n of a packed key stream (the reference's bit order)
__device__ __forceinline__ uint32_t get_code_ref(const uint8_t* packed, size_t n, int bits, size_t nbytes) {
  const size_t p = n * (size_t)bits, b0 = p >> 3;
  const uint32_t win = ((uint32_t)packed[b0] << 8) | (b0 + 1 < nbytes ? packed[b0 + 1] : 0u);
  const int o = (int)(p & 7);
  uint32_t c = 0;
  for (int k = 0; k < bits; ++k) c |= ((win >> (15 - o - k)) & 1u) << k;
  return c;
}

struct KeyBlockArgs {
  tqk_block_desc d;
  const void* x;
  const float* zp;
  uint8_t* packed;
  float* scale;
  float* zero;
  uint32_t* out_pos;
  uint16_t* out_val;
  int32_t* out_count;
  int thr_pre;     // the thresholds were left in out_pos by tqk_key_block_thresholds
  int codes_post;  // the 4-bit codes are written by tqk_key_block_codes4 afterwards
};

// The outlier thresholds of tqk_key_block ahead of it, spread over the chip:
// one workgroup per (b, h) and 64 channels, a lane per channel and 16 waves
// over interleaved token rows (each load one 128-byte row piece).  The same
// search as tqk_key_block's threshold threads: T is the largest fp32
// magnitude pattern with #{ |x_s| >= T } >= k, found two bits a pass, each
// pass's counts exact integer sums of the 16 waves' counts.  T is left in the
// first D entries of the (b, h)'s side-list row (out_pos), which
// tqk_key_block reads before it writes that row.
template <int D>
__global__ __launch_bounds__(1024) void tqk_key_block_thresholds(KeyBlockArgs a) {
  constexpr int W = 16;
  const tqk_block_desc& d = a.d;
  const int bh = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = blockIdx.y * 64 + lane;
  const int S = d.tokens, f32 = d.input_f32, kout = d.outliers_per_channel;
  const size_t base = (size_t)bh * S * D + j;
  // Two bits a pass (bits 30..1 in pairs, then bit 0): the counts of the
  // three candidates T | d << sh (d = 1, 2, 3) fall with d, so the largest d
  // whose count reaches k is what two one-bit passes would pick.
  __shared__ int cnt_s[2][3][W][64];
  uint32_t T = 0;
  int par = 0;
  for (int sh = 29; sh >= -1; sh -= 2, par ^= 1) {
    const bool two = sh >= 1;
    const int shift = two ? sh : 0;
    const uint32_t c1 = T | (1u << shift), c2 = T | (2u << shift), c3 = T | (3u << shift);
    int n1 = 0, n2 = 0, n3 = 0;
    for_tokens<D>(a.x, f32, base, w, S, W, [&](int, float xv) {
      const uint32_t u = __float_as_uint(fabsf(xv));
      n1 += u >= c1;
      n2 += u >= c2;
      n3 += u >= c3;
    });
    // (two count buffers: a wave that runs ahead writes the other one; the
    // next write to this one follows the next pass's barrier)
    cnt_s[par][0][w][lane] = n1;
    cnt_s[par][1][w][lane] = n2;
    cnt_s[par][2][w][lane] = n3;
    __syncthreads();
    int t1 = 0, t2 = 0, t3 = 0;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      t1 += cnt_s[par][0][v][lane];
      t2 += cnt_s[par][1][v][lane];
      t3 += cnt_s[par][2][v][lane];
    }
    const uint32_t dsel = two ? (t3 >= kout ? 3u : t2 >= kout ? 2u : t1 >= kout ? 1u : 0u)
                              : (t1 >= kout ? 1u : 0u);
    T |= dsel << shift;
  }
  if (w == 0) a.out_pos[(size_t)bh * d.outlier_cap + j] = T;
}

// one workgroup of 2 * D threads per (b, h)
template <int D>
__global__ __launch_bounds__(2 * D) void tqk_key_block(KeyBlockArgs a) {
  constexpr int T = 2 * D;  // threads
  const tqk_block_desc& d = a.d;
  const int bh = blockIdx.x, h = bh % d.n_heads, tid = threadIdx.x;
  const int S = d.tokens, f32 = d.input_f32, kout = d.outliers_per_channel;
  const size_t base = (size_t)bh * S * D;
  auto X = [&](int s, int j) { return load_x(a.x, f32, base + (size_t)s * D + j); };

  __shared__ float cent_s[D][17];  // per-channel grid (uniform: min, scale)
  __shared__ float thr_s[D];       // outlier threshold magnitude per channel
  __shared__ int32_t wsum_s[T / 64];

  // ---- per-channel statistics (threads 0..D-1) and thresholds (D..2D-1)
  if (tid < D) {
    const int j = tid;
    if (d.key_grid == 1) {
      float mn = X(0, j), mx = mn;
      bool nan = (mn != mn);
      for_tokens<D>(a.x, f32, base + j, 1, S, 1, [&](int, float xv) {
        nan |= (xv != xv);
        mn = fminf(mn, xv);
        mx = fmaxf(mx, xv);
      });
      const float sc = nan ? __builtin_nanf("") : __fdiv_rn(fmaxf(__fsub_rn(mx, mn), 1e-8f),
                                                            (float)((1 << d.bits) - 1));
      if (nan) mn = __builtin_nanf("");
      cent_s[j][0] = mn;
      cent_s[j][1] = sc;
      a.scale[(size_t)bh * D + j] = sc;
      a.zero[(size_t)bh * D + j] = mn;
    } else {
      float mu;
      if (d.zero_point == 2) {
        mu = a.zp[(size_t)h * D + j];
      } else {
        float acc = 0.0f;  // in token order
        for_tokens<D>(a.x, f32, base + j, 0, S, 1, [&](int, float xv) { acc = __fadd_rn(acc, xv); });
        mu = (float)((double)acc / (double)S);
        if (d.zero_point == 1) mu = __fmul_rn(mu, dc_channel(d, j) ? 1.0f : 0.0f);
      }
      float amax = 0.0f;
      bool nan = (mu != mu);
      for_tokens<D>(a.x, f32, base + j, 0, S, 1, [&](int, float xv) {
        const float dv = fabsf(__fsub_rn(xv, mu));
        nan |= (dv != dv);
        amax = fmaxf(amax, dv);
      });
      amax = nan ? __builtin_nanf("") : fmaxf(amax, 1e-8f);
#pragma unroll
      for (int l = 0; l < 16; ++l) cent_s[j][l] = __fadd_rn(mu, __fmul_rn(amax, kNF4[l]));
      a.scale[(size_t)bh * D + j] = amax;
      a.zero[(size_t)bh * D + j] = mu;
    }
  } else if (tid < 2 * D && kout > 0 && kout < S) {
    // k-th largest |x| as the largest fp32 magnitude pattern T with
    // #{ |x_s| >= T } >= k (NaN patterns order above inf, as np.partition does)
    const int j = tid - D;
    uint32_t T = 0;
    if (a.thr_pre) {
      T = a.out_pos[(size_t)bh * d.outlier_cap + j];
    } else {
      for (int bit = 30; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        int cnt = 0;
        for (int s = 0; s < S; ++s) cnt += (__float_as_uint(fabsf(X(s, j))) >= cand);
        if (cnt >= kout) T = cand;
      }
    }
    thr_s[j] = __uint_as_float(T);
  }
  __syncthreads();

  // ---- codes of 3- and 2-bit (uniform) keys: one token row per thread
  if (d.bits != 4) {
    const int bits = d.bits, rwords = D * bits / 32;  // D * bits / 8 bytes per token
    const float qmax = (float)((1 << bits) - 1);
    for (int s = tid; s < S; s += T) {
      uint32_t rw[D / 8] = {0u};
      for (int j = 0; j < D; ++j) {
        const float r = __builtin_rintf(__fdiv_rn(__fsub_rn(X(s, j), cent_s[j][0]), cent_s[j][1]));
        put_code_ref(rw, j, bits, (uint32_t)fminf(fmaxf(r, 0.0f), qmax));
      }
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.packed + ((size_t)bh * S + s) * (size_t)(D * bits / 8));
      for (int w = 0; w < rwords; ++w) dst[w] = rw[w];
    }
  }
  // ---- 4-bit codes: thread = (channel pair, token slice), one byte per (token, pair)
  else if (!a.codes_post) {
    const int jp = tid % (D / 2), sq = tid / (D / 2);  // four token slices
    const int per = (S + 3) / 4, s0 = sq * per, s1 = min(S, s0 + per);
    uint8_t* out = a.packed + base / 2 + jp;
    if (d.key_grid == 1) {
      const float mn0 = cent_s[2 * jp][0], sc0 = cent_s[2 * jp][1];
      const float mn1 = cent_s[2 * jp + 1][0], sc1 = cent_s[2 * jp + 1][1];
      for_token_pairs<D>(a.x, f32, base + 2 * jp, s0, s1, [&](int s, float x0, float x1) {
        const float r0 = __builtin_rintf(__fdiv_rn(__fsub_rn(x0, mn0), sc0));
        const float r1 = __builtin_rintf(__fdiv_rn(__fsub_rn(x1, mn1), sc1));
        const uint32_t b0 = (uint32_t)fminf(fmaxf(r0, 0.0f), 15.0f);
        const uint32_t b1 = (uint32_t)fminf(fmaxf(r1, 0.0f), 15.0f);
        out[(size_t)s * (D / 2)] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
      });
    } else {
      float c0[16], c1[16];
#pragma unroll
      for (int l = 0; l < 16; ++l) {
        c0[l] = cent_s[2 * jp][l];
        c1[l] = cent_s[2 * jp + 1][l];
      }
      for_token_pairs<D>(a.x, f32, base + 2 * jp, s0, s1, [&](int s, float x0, float x1) {
        int b0 = 0, b1 = 0;
        float d0 = fabsf(__fsub_rn(x0, c0[0])), d1 = fabsf(__fsub_rn(x1, c1[0]));
#pragma unroll
        for (int l = 1; l < 16; ++l) {
          const float e0 = fabsf(__fsub_rn(x0, c0[l])), e1 = fabsf(__fsub_rn(x1, c1[l]));
          // np.argmin: strictly smaller wins; the first NaN wins over any number
          if (e0 < d0 || (e0 != e0 && d0 == d0)) { d0 = e0; b0 = l; }
          if (e1 < d1 || (e1 != e1 && d1 == d1)) { d1 = e1; b1 = l; }
        }
        out[(size_t)s * (D / 2)] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
      });
    }
  }

  // ---- outlier side-list in (s, j) order: wave w owns a contiguous token
  // range and a lane one channel of each 64-channel piece of a token row (one
  // coalesced row piece per load); the pieces' ballots count the wave's
  // entries, its offset comes from the waves before it, and the entries are
  // written at offset + the lanes before them in the ballot
  if (kout > 0) {
    const bool all = kout >= S;
    constexpr int NWV = T / 64, NC = D / 64;
    const int wv = tid >> 6, ln = tid & 63;
    const int chunk = (S + NWV - 1) / NWV;
    const int s0 = min(S, wv * chunk), s1 = min(S, s0 + chunk);
    float th[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) th[c] = thr_s[c * 64 + ln];
    int cnt = 0;  // the same in every lane of the wave
#pragma unroll
    for (int c = 0; c < NC; ++c)
      for_tokens<D>(a.x, f32, base + c * 64 + ln, s0, s1, 1, [&](int, float xv) {
        cnt += __popcll(__ballot(all || fabsf(xv) >= th[c]));
      });
    if (ln == 0) wsum_s[wv] = cnt;
    __syncthreads();
    int off = 0, total = 0;
    for (int w = 0; w < NWV; ++w) {
      if (w < wv) off += wsum_s[w];
      total += wsum_s[w];
    }
    if (tid == 0) a.out_count[bh] = total;
    const size_t lb = (size_t)bh * d.outlier_cap;
    const uint64_t before = (1ull << ln) - 1ull;  // the lanes ahead of this one
    for (int s4 = s0; s4 < s1 && off < d.outlier_cap; s4 += 4) {
      float xr[4][NC];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int c = 0; c < NC; ++c) xr[u][c] = X(min(s4 + u, s1 - 1), c * 64 + ln);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s4 + u;
        if (s >= s1) break;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int j = c * 64 + ln;
          const float xv = xr[u][c];
          const bool hit = all || fabsf(xv) >= th[c];
          const uint64_t m = __ballot(hit);
          const int at = off + __popcll(m & before);
          if (hit && at < d.outlier_cap) {
            a.out_pos[lb + at] = (uint32_t)s * D + (uint32_t)j;
            a.out_val[lb + at] = f2h(xv);  // fp16, round to nearest even
          }
          off += __popcll(m);
        }
      }
    }
  } else if (tid == 0) {
    a.out_count[bh] = 0;
  }
}

// The 4-bit codes of tqk_key_block over the chip: a workgroup per (b, h) and
// 256 tokens, thread = (channel pair, token slice).  The levels are rebuilt
// from the scale and zero point tqk_key_block stored, with its arithmetic
// (NF4: mean + amax * level; uniform: min and step), so the codes are its.
template <int D>
__global__ __launch_bounds__(256) void tqk_key_block_codes4(KeyBlockArgs a) {
  constexpr int NPR = D / 2, NS = 256 / NPR, TOK = 256, PER = TOK / NS;
  const tqk_block_desc& d = a.d;
  const int bh = blockIdx.x, tid = threadIdx.x, jp = tid % NPR, sq = tid / NPR;
  const int S = d.tokens, f32 = d.input_f32;
  const size_t base = (size_t)bh * S * D;
  const int t0 = blockIdx.y * TOK, t1 = min(S, t0 + TOK);
  const int s0 = min(t1, t0 + sq * PER), s1 = min(t1, s0 + PER);
  uint8_t* out = a.packed + base / 2 + jp;
  const size_t cj = (size_t)bh * D + 2 * jp;
  const float sc0 = a.scale[cj], z0 = a.zero[cj], sc1 = a.scale[cj + 1], z1 = a.zero[cj + 1];
  if (d.key_grid == 1) {
    for_token_pairs<D>(a.x, f32, base + 2 * jp, s0, s1, [&](int s, float x0, float x1) {
      const float r0 = __builtin_rintf(__fdiv_rn(__fsub_rn(x0, z0), sc0));
      const float r1 = __builtin_rintf(__fdiv_rn(__fsub_rn(x1, z1), sc1));
      const uint32_t b0 = (uint32_t)fminf(fmaxf(r0, 0.0f), 15.0f);
      const uint32_t b1 = (uint32_t)fminf(fmaxf(r1, 0.0f), 15.0f);
      out[(size_t)s * (D / 2)] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
    });
  } else {
    float c0[16], c1[16];
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      c0[l] = __fadd_rn(z0, __fmul_rn(sc0, kNF4[l]));
      c1[l] = __fadd_rn(z1, __fmul_rn(sc1, kNF4[l]));
    }
    for_token_pairs<D>(a.x, f32, base + 2 * jp, s0, s1, [&](int s, float x0, float x1) {
      int b0 = 0, b1 = 0;
      float d0 = fabsf(__fsub_rn(x0, c0[0])), d1 = fabsf(__fsub_rn(x1, c1[0]));
#pragma unroll
      for (int l = 1; l < 16; ++l) {
        const float e0 = fabsf(__fsub_rn(x0, c0[l])), e1 = fabsf(__fsub_rn(x1, c1[l]));
        // np.argmin: strictly smaller wins; the first NaN wins over any number
        if (e0 < d0 || (e0 != e0 && d0 == d0)) { d0 = e0; b0 = l; }
        if (e1 < d1 || (e1 != e1 && d1 == d1)) { d1 = e1; b1 = l; }
      }
      out[(size_t)s * (D / 2)] = (uint8_t)((rev4(b0) << 4) | rev4(b1));
    });
  }
}

struct ValueBlockArgs {
  tqk_block_desc d;
  const void* x;
  const float* pi;
  const float* vbnd;
  uint8_t* packed;
  float* norms;
};

// 64 tokens of one (b, h) per workgroup.  Four threads per token compute the
// norm in the reference's pairwise order and stage the normalised row in LDS;
// then the rotation as in the group encode (DPP row broadcasts of register-
// held row slices, a column of Pi_T per lane).
template <int VB, int D>
__global__ __launch_bounds__(kVbThreads) void tqk_value_block(ValueBlockArgs a) {
  constexpr int VROW = D * VB / 8;
  const tqk_block_desc& d = a.d;
  const int S = d.tokens, bh = blockIdx.y, t0 = blockIdx.x * kVbTokens, tid = threadIdx.x;
  const int nb = min(kVbTokens, S - t0);
  const size_t tok0 = (size_t)bh * S + t0;  // flat token index of the first token
  __shared__ __align__(16) float u_s[kVbTokens][D];
  __shared__ uint8_t vc_s[kVbTokens][D];

  {
    const int tt = tid >> 2, q = tid & 3;
    if (tt < nb) {
      const size_t row = (tok0 + tt) * D;
      float x0[D / 8], x1[D / 8];
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {  // channels 8m + 2q, 8m + 2q + 1
        x0[m] = load_x(a.x, d.input_f32, row + 8 * m + 2 * q);
        x1[m] = load_x(a.x, d.input_f32, row + 8 * m + 2 * q + 1);
      }
      const float ss = pairwise_sumsq<D>(x0, x1, q);
      const float nrm = __builtin_sqrtf(ss);  // correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt)
      const float safe = fmaxf(nrm, 1e-30f);
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        u_s[tt][8 * m + 2 * q] = __fdiv_rn(x0[m], safe);
        u_s[tt][8 * m + 2 * q + 1] = __fdiv_rn(x1[m], safe);
      }
      if (q == 0) a.norms[tok0 + tt] = nrm;
    }
  }
  // rotation: wave w owns the rotated channels [16w + 128p, +16) of pass p,
  // lane l column e = 16w + 128p + (l & 15) of Pi_T (row e of Pi) in
  // registers; each 16-lane row takes one token of a 4-token step, holds
  // eight channels of its normalised row and broadcasts them to the row by
  // DPP (rotate_codes, no LDS broadcast reads)
  const int lane = tid & 63, wv = tid >> 6;
  float bnd[15];
#pragma unroll
  for (int k = 0; k < (1 << VB) - 1; ++k) bnd[k] = a.vbnd[k];
  __syncthreads();
  for (int e0 = 16 * wv; e0 < D; e0 += 16 * (kVbThreads / 64))
    rotate_codes<D, VB>(a.pi, u_s, nb, e0 + (lane & 15), lane, bnd, vc_s);
  __syncthreads();
  // the reference's little-endian bit stream, one token per thread
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
    uint32_t* dst = reinterpret_cast<uint32_t*>(a.packed + (tok0 + tid) * VROW);
#pragma unroll
    for (int k = 0; k < VROW / 4; ++k) dst[k] = outw[k];
  }
}

struct KeyDequantArgs {
  tqk_block_desc d;
  const uint8_t* packed;
  const float* scale;
  const float* zero;
  float* out;
};

// one thread per code byte (two channels): zero + scale * level[code]; 3- and
// 2-bit keys one thread per code
__global__ __launch_bounds__(kKbThreads) void tqk_key_block_dequant(KeyDequantArgs a) {
  const tqk_block_desc& d = a.d;
  const int D = d.head_dim;
  if (d.bits != 4) {
    const size_t n = (size_t)d.batch * d.n_heads * d.tokens * D;
    const size_t i = (size_t)blockIdx.x * kKbThreads + threadIdx.x;
    if (i >= n) return;
    const size_t bh = i / ((size_t)d.tokens * D);
    const int j = (int)(i % D);
    const uint32_t c = get_code_ref(a.packed, i, d.bits, (n * d.bits + 7) / 8);
    a.out[i] = __fadd_rn(__fmul_rn(a.scale[bh * D + j], (float)c), a.zero[bh * D + j]);
    return;
  }
  const size_t n = (size_t)d.batch * d.n_heads * d.tokens * (D / 2);
  const size_t i = (size_t)blockIdx.x * kKbThreads + threadIdx.x;
  if (i >= n) return;
  const size_t bh = i / ((size_t)d.tokens * (D / 2));
  const int j0 = 2 * (int)(i % (D / 2));
  const uint32_t byte = a.packed[i];
  const float* sc = a.scale + bh * D;
  const float* zr = a.zero + bh * D;
  a.out[2 * i] = __fadd_rn(__fmul_rn(sc[j0], key_level(d.key_grid, rev4(byte >> 4))), zr[j0]);
  a.out[2 * i + 1] = __fadd_rn(__fmul_rn(sc[j0 + 1], key_level(d.key_grid, rev4(byte & 15u))), zr[j0 + 1]);
}

// the side-list overwrite (after the dense pass on the same stream); an index
// outside [0, total) is skipped here and reported by the host-side check
__global__ __launch_bounds__(kKbThreads) void tqk_key_block_outliers(float* out, int n,
                                                                   int64_t total,
                                                                   const int32_t* idx,
                                                                   const uint16_t* val) {
  const int i = blockIdx.x * kKbThreads + threadIdx.x;
  if (i < n) {
    const int64_t p = idx[i];
    if (p >= 0 && p < total) out[p] = h2f(val[i]);
  }
}

struct ValueDequantArgs {
  tqk_block_desc d;
  const uint8_t* packed;
  const float* norms;
  const float* pi;
  const float* vcent;
  float* out;
};

// one thread per token: y = vcent[code]; x_e = sequential over j of y_j * Pi[j][e]; x * norm
template <int VB, int D>
__global__ __launch_bounds__(kKbThreads) void tqk_value_block_dequant(ValueDequantArgs a) {
  constexpr int VROW = D * VB / 8;
  const tqk_block_desc& d = a.d;
  const size_t n = (size_t)d.batch * d.n_heads * d.tokens;
  const size_t t = (size_t)blockIdx.x * kKbThreads + threadIdx.x;
  if (t >= n) return;
  const uint8_t* vr = a.packed + t * VROW;
  float y[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int bitpos = j * VB;
    const uint32_t w = vr[bitpos >> 3] | ((uint32_t)vr[min((bitpos >> 3) + 1, VROW - 1)] << 8);
    y[j] = a.vcent[(w >> (bitpos & 7)) & ((1u << VB) - 1)];
  }
  const float nrm = a.norms[t];
  float* o = a.out + t * D;
  for (int e = 0; e < D; ++e) {
    float x = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) x = __fadd_rn(x, __fmul_rn(y[j], a.pi[j * D + e]));
    o[e] = __fmul_rn(x, nrm);
  }
}

int check_block(const tqk_block_desc* d, bool key) {
  if (!d) return TQK_EINVAL;
  if (!head_dim_ok(d->head_dim)) return TQK_EUNSUPPORTED;
  if (d->batch <= 0 || d->n_heads <= 0 || d->tokens <= 0) return TQK_EINVAL;
  if ((long long)d->batch * d->n_heads * d->tokens * d->head_dim >= (1LL << 40)) return TQK_EINVAL;
  if (key) {
    if (d->bits < 2 || d->bits > 4) return TQK_EUNSUPPORTED;
    if (d->key_grid != 0 && d->key_grid != 1) return TQK_EINVAL;
    if (d->bits != 4 && d->key_grid != 1) return TQK_EUNSUPPORTED;  // NF4 is 4-bit
    if (d->zero_point < 0 || d->zero_point > 2 || (d->zero_point != 0 && d->key_grid != 0))
      return TQK_EINVAL;
    if (d->outliers_per_channel < 0 || d->outlier_cap < 0) return TQK_EINVAL;
    // side-list positions s * D + j are 32-bit
    if ((long long)d->tokens * d->head_dim >= (1LL << 32)) return TQK_EUNSUPPORTED;
  } else if (d->bits < 2 || d->bits > 4) {
    return TQK_EUNSUPPORTED;
  }
  return TQK_OK;
}

// one kernel instance per (bits, head_dim)
template <int D>
void launch_value(int vb, dim3 grid, hipStream_t st, const ValueBlockArgs& a) {
  if (vb == 2)
    hipLaunchKernelGGL((tqk_value_block<2, D>), grid, dim3(kVbThreads), 0, st, a);
  else if (vb == 3)
    hipLaunchKernelGGL((tqk_value_block<3, D>), grid, dim3(kVbThreads), 0, st, a);
  else
    hipLaunchKernelGGL((tqk_value_block<4, D>), grid, dim3(kVbThreads), 0, st, a);
}
template <int D>
void launch_value(int vb, dim3 grid, hipStream_t st, const ValueDequantArgs& a) {
  if (vb == 2)
    hipLaunchKernelGGL((tqk_value_block_dequant<2, D>), grid, dim3(kKbThreads), 0, st, a);
  else if (vb == 3)
    hipLaunchKernelGGL((tqk_value_block_dequant<3, D>), grid, dim3(kKbThreads), 0, st, a);
  else
    hipLaunchKernelGGL((tqk_value_block_dequant<4, D>), grid, dim3(kKbThreads), 0, st, a);
}

}  // namespace

extern "C" {

int tqk_encode_key_block(const tqk_block_desc* d, const void* x, const float* zp, uint8_t* packed,
                         float* scale, float* zero, uint32_t* out_pos, uint16_t* out_val,
                         int32_t* out_count, void* stream) {
  int rc = check_block(d, true);
  if (rc != TQK_OK) return rc;
  if (!x || !packed || !scale || !zero || !out_count) return TQK_EINVAL;
  if (d->key_grid == 0 && d->zero_point == 2 && !zp) return TQK_EINVAL;
  if (d->outliers_per_channel > 0 && d->outlier_cap > 0 && (!out_pos || !out_val)) return TQK_EINVAL;
  KeyBlockArgs a{*d, x, zp, packed, scale, zero, out_pos, out_val, out_count, 0};
  const dim3 grid(d->batch * d->n_heads);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // thresholds ahead, over the chip, where the side-list row can hold them
  if (d->outliers_per_channel > 0 && d->outliers_per_channel < d->tokens &&
      d->outlier_cap >= d->head_dim) {
    a.thr_pre = 1;
    const dim3 tgrid(d->batch * d->n_heads, d->head_dim / 64);
    if (d->head_dim == 64)
      hipLaunchKernelGGL(tqk_key_block_thresholds<64>, tgrid, dim3(1024), 0, st, a);
    else if (d->head_dim == 128)
      hipLaunchKernelGGL(tqk_key_block_thresholds<128>, tgrid, dim3(1024), 0, st, a);
    else
      hipLaunchKernelGGL(tqk_key_block_thresholds<256>, tgrid, dim3(1024), 0, st, a);
  }
  // 4-bit codes afterwards, over the chip (a workgroup per 256 tokens)
  const int n_tok_blocks = (d->tokens + 255) / 256;
  a.codes_post = d->bits == 4 && n_tok_blocks <= 65535;
  if (d->head_dim == 64)
    hipLaunchKernelGGL(tqk_key_block<64>, grid, dim3(128), 0, st, a);
  else if (d->head_dim == 128)
    hipLaunchKernelGGL(tqk_key_block<128>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(tqk_key_block<256>, grid, dim3(512), 0, st, a);
  if (a.codes_post) {
    const dim3 cgrid(d->batch * d->n_heads, n_tok_blocks);
    if (d->head_dim == 64)
      hipLaunchKernelGGL(tqk_key_block_codes4<64>, cgrid, dim3(256), 0, st, a);
    else if (d->head_dim == 128)
      hipLaunchKernelGGL(tqk_key_block_codes4<128>, cgrid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(tqk_key_block_codes4<256>, cgrid, dim3(256), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int tqk_encode_value_block(const tqk_block_desc* d, const void* x, const float* pi,
                           const float* vbnd, uint8_t* packed, float* norms, void* stream) {
  int rc = check_block(d, false);
  if (rc != TQK_OK) return rc;
  if (!x || !pi || !vbnd || !packed || !norms) return TQK_EINVAL;
  ValueBlockArgs a{*d, x, pi, vbnd, packed, norms};
  const dim3 grid((d->tokens + kVbTokens - 1) / kVbTokens, d->batch * d->n_heads);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (d->head_dim == 64)
    launch_value<64>(d->bits, grid, st, a);
  else if (d->head_dim == 128)
    launch_value<128>(d->bits, grid, st, a);
  else
    launch_value<256>(d->bits, grid, st, a);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int tqk_dequant_key_block(const tqk_block_desc* d, const uint8_t* packed, const float* scale,
                          const float* zero, int32_t n_out, const int32_t* out_idx,
                          const uint16_t* out_val, float* out, void* stream) {
  int rc = check_block(d, true);
  if (rc != TQK_OK) return rc;
  if (!packed || !scale || !zero || !out || n_out < 0 || (n_out > 0 && (!out_idx || !out_val)))
    return TQK_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t total = (size_t)d->batch * d->n_heads * d->tokens * d->head_dim;
  const size_t n = d->bits == 4 ? total / 2 : total;  // threads: code bytes, or codes
  KeyDequantArgs a{*d, packed, scale, zero, out};
  hipLaunchKernelGGL(tqk_key_block_dequant, dim3((unsigned)((n + kKbThreads - 1) / kKbThreads)),
                     dim3(kKbThreads), 0, st, a);
  if (n_out > 0)
    hipLaunchKernelGGL(tqk_key_block_outliers, dim3((n_out + kKbThreads - 1) / kKbThreads),
                       dim3(kKbThreads), 0, st, out, n_out, (int64_t)total, out_idx, out_val);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

int tqk_dequant_value_block(const tqk_block_desc* d, const uint8_t* packed, const float* norms,
                            const float* pi, const float* vcent, float* out, void* stream) {
  int rc = check_block(d, false);
  if (rc != TQK_OK) return rc;
  if (!packed || !norms || !pi || !vcent || !out) return TQK_EINVAL;
  const size_t n = (size_t)d->batch * d->n_heads * d->tokens;
  ValueDequantArgs a{*d, packed, norms, pi, vcent, out};
  const dim3 grid((unsigned)((n + kKbThreads - 1) / kKbThreads));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (d->head_dim == 64)
    launch_value<64>(d->bits, grid, st, a);
  else if (d->head_dim == 128)
    launch_value<128>(d->bits, grid, st, a);
  else
    launch_value<256>(d->bits, grid, st, a);
  return hipGetLastError() == hipSuccess ? TQK_OK : TQK_EHIP;
}

}  // extern "C"
