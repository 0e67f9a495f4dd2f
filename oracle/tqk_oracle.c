/*
 * Scalar C restatement of the TurboQuant Pro encode (quantize-on-flush) with
 * every floating-point operation in the order NumPy performs it.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ through ctypes to pin the
 * operation order that the gfx950 encode kernel follows.  Never linked into
 * the product library.  Build: see oracle/Makefile (-O2 -ffp-contract=off).
 *
 * Keys, one group (H, S, D) fp32, turboquant_pro/per_channel_kv.py:269-401:
 *   mean  = fl(sequential token-order sum) / S          (np.mean over axis 2)
 *   amax  = max(max_s |fl(x - mean)|, 1e-8)
 *   cent  = fl(mean + fl(amax * NF4[l]))
 *   code  = first argmin_l |fl(x - cent[l])|
 *   outliers: threshold = k-th largest |x| per (h, j); keep |x| >= threshold,
 *   flat C-order index over (1, H, S, D).
 * Values, one vector (D) fp32, turboquant_pro/core.py:569-606:
 *   norm  = sqrt of NumPy's pairwise sum of squares (8 strided accumulators
 *           per run of <= 128, combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7));
 *           a longer row is its halves' sums added)
 *   u     = v / max(norm, 1e-30)
 *   y_e   = sequential-over-d fl(y + fl(u_d * PiT[d][e]))   (np.einsum, no FMA)
 *   code  = #{ b < y }                                      (searchsorted left)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};

static int cmp_float(const void* a, const void* b) {
  float x = *(const float*)a, y = *(const float*)b;
  return (x > y) - (x < y);
}

/* NumPy's pairwise summation of a contiguous float32 run
 * (numpy/_core/src/umath/loops_utils.h.src, pairwise_sum): n < 8 sequential;
 * n <= 128 eight strided accumulators combined as a tree, then the remainder;
 * longer runs split at n / 2 rounded down to a multiple of 8, halves summed
 * apart and added. */
static float pairwise_sum_f32(const float* a, int n) {
  if (n < 8) {
    float r = 0.0f;  /* numpy starts from -0.0 for n<8 then adds; equal for our use */
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  if (n > 128) {
    int n2 = n / 2;
    n2 -= n2 % 8;
    return pairwise_sum_f32(a, n2) + pairwise_sum_f32(a + n2, n - n2);
  }
  float r[8];
  for (int k = 0; k < 8; ++k) r[k] = a[k];
  int i;
  for (i = 8; i < n - (n % 8); i += 8)
    for (int k = 0; k < 8; ++k) r[k] += a[i + k];
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}

/* Keys of one group.  x: (H, S, D) fp32.  codes: (H, S, D).  scale/mean: (H, D).
 * k_out: outliers kept per channel (<= 0: none).  oidx: capacity H*S*D.
 * Returns the outlier count. */
int tqo_encode_keys(const float* x, int H, int S, int D, int k_out, uint8_t* codes,
                    float* scale, float* mean, int32_t* oidx) {
  float* col = (float*)malloc(sizeof(float) * (size_t)S);
  float* thr = (float*)malloc(sizeof(float) * (size_t)H * D);
  for (int h = 0; h < H; ++h) {
    for (int j = 0; j < D; ++j) {
      const float* xj = x + (size_t)h * S * D + j;
      float acc = 0.0f;
      for (int s = 0; s < S; ++s) acc = acc + xj[(size_t)s * D];
      /* np.mean divides the fp32 sum by an intp count: float64 division, then fp32 */
      float mu = (float)((double)acc / (double)S);
      float amax = 0.0f;
      for (int s = 0; s < S; ++s) {
        float d = fabsf(xj[(size_t)s * D] - mu);
        if (d > amax) amax = d;
      }
      if (amax < 1e-8f) amax = 1e-8f;
      float cent[16];
      for (int l = 0; l < 16; ++l) {
        float t = amax * kNF4[l];
        cent[l] = mu + t;
      }
      for (int s = 0; s < S; ++s) {
        float xv = xj[(size_t)s * D];
        int best = 0;
        float bd = fabsf(xv - cent[0]);
        for (int l = 1; l < 16; ++l) {
          float d = fabsf(xv - cent[l]);
          if (d < bd) { bd = d; best = l; }
        }
        codes[((size_t)h * S + s) * D + j] = (uint8_t)best;
      }
      scale[h * D + j] = amax;
      mean[h * D + j] = mu;
      if (k_out > 0 && k_out < S) {
        for (int s = 0; s < S; ++s) col[s] = fabsf(xj[(size_t)s * D]);
        qsort(col, (size_t)S, sizeof(float), cmp_float);
        thr[h * D + j] = col[S - k_out];
      } else {
        thr[h * D + j] = 0.0f;  /* k >= S keeps everything */
      }
    }
  }
  int n = 0;
  if (k_out > 0) {
    for (int h = 0; h < H; ++h)
      for (int s = 0; s < S; ++s)
        for (int j = 0; j < D; ++j) {
          size_t f = ((size_t)h * S + s) * D + j;
          if (fabsf(x[f]) >= thr[h * D + j]) oidx[n++] = (int32_t)f;
        }
  }
  free(col);
  free(thr);
  return n;
}

/* Values.  v: (N, D) fp32 rows.  pi_t: (D, D) row-major.  bnd: nb boundaries. */
void tqo_encode_values(const float* v, int N, int D, const float* pi_t, const float* bnd,
                       int nb, uint8_t* codes, float* norms) {
  float* sq = (float*)malloc(sizeof(float) * (size_t)D);
  float* u = (float*)malloc(sizeof(float) * (size_t)D);
  for (int r = 0; r < N; ++r) {
    const float* x = v + (size_t)r * D;
    for (int d = 0; d < D; ++d) sq[d] = x[d] * x[d];
    float nrm = sqrtf(pairwise_sum_f32(sq, D));
    float safe = nrm > 1e-30f ? nrm : 1e-30f;
    for (int d = 0; d < D; ++d) u[d] = x[d] / safe;
    for (int e = 0; e < D; ++e) {
      float y = 0.0f;
      for (int d = 0; d < D; ++d) {
        float p = u[d] * pi_t[(size_t)d * D + e];
        y = y + p;
      }
      int c = 0;
      for (int i = 0; i < nb; ++i) c += (bnd[i] < y);
      codes[(size_t)r * D + e] = (uint8_t)c;
    }
    norms[r] = nrm;
  }
  free(sq);
  free(u);
}
