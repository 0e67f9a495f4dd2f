/*
 * tqk.h -- C ABI of the MI355X (gfx950) TurboQuant Pro KV-cache kernels.
 *
 * One hot path: the two-tier TurboQuant KV cache (fp16 hot window + flushed
 * groups of per-channel 4-bit keys -- asym-NF4 with a calibrated, sparse or
 * bias zero point, or uniform -- with an fp16 outlier side-list, and
 * PolarQuant 2/3/4-bit values) and the fused decode-step attention over it.
 *
 * Conventions
 *   - Every pointer is a DEVICE pointer unless its comment says host.
 *   - The caller owns every buffer (including the decode workspace); the
 *     library allocates nothing per call.
 *   - Every entry point returns an int status (TQK_OK or an error code) and
 *     never throws or aborts across the ABI.
 *   - Work is enqueued on the given HIP stream (hipStream_t passed as void*;
 *     NULL = the default stream) and is stream-ordered.
 *   - fp16 data is passed as uint16_t bit patterns (IEEE binary16); K/V/q
 *     buffers typed void* are fp16, or fp32 when the descriptor's input_f32 is 1.
 *
 * Storage layout in HBM (one cache pool = one attention layer):
 *   kcodes [n_kv_heads][n_pages][page_tokens][head_dim/2]     u8   (storage of record)
 *   vcodes [n_kv_heads][n_pages][page_tokens][head_dim*vb/8]  u8   (storage of record, see below)
 *   vnorm  [n_kv_heads][n_pages][page_tokens]                 f32
 *   (head-major: a head's pages are one contiguous region, so consecutive
 *   physical pages of a head are adjacent in memory)
 *   gscale [num_gslots][n_kv_heads][head_dim]                 f32  (nf4_scale)
 *   gmean  [num_gslots][n_kv_heads][head_dim]                 f32  (nf4_mean)
 *   ocount [num_gslots][n_kv_heads][8]  i32 cumulative outlier counts at tokens 32,64,..,256 (last = total)
 *   oent   [num_gslots][n_kv_heads][outlier_cap]              u32  ((s*D + j) | fp16 << 16)
 *   hot_k, hot_v [batch][n_kv_heads][hot_ring][head_dim]      fp16 (fp32 when input_f32) ring,
 *                                                             token t at t % hot_ring
 *   block_table [batch][max_pages_per_seq]   i32 physical page of logical page t / page_tokens
 *   group_table [batch][max_groups_per_seq]  i32 group slot of group t / group_tokens
 * The K and V rows are the reference's packed layouts
 * (turboquant_pro/per_channel_kv.py:87-93 and turboquant_pro/core.py:350-398):
 * the key bytes of one (group, head) in page order are the reference
 * container's `indices` slice for that head, except that (fp16 caches) every
 * position held in oent stores the code whose level is 0 -- NF4's code 7 (nibble 0xE) for
 * key_grid 0, code 0 for key_grid 1 -- so that the dense part of a decode
 * contributes exactly gmean there and the side-list adds val - gmean (exact
 * only because the stored level's reconstruction equals gmean; fp32 caches
 * keep the reference's codes there and the VALU decode subtracts the dense
 * level it reads).  The
 * reference's code at such a position is the nearest level to the stored
 * fp16 value (recomputed on export).  Value bytes are the reference's
 * per-token pack when head_dim != 128, input_f32, page_tokens % 16 != 0 or
 * group_tokens % 32 != 0; otherwise
 * each 16-token tile of a page holds 64 units of head_dim*vb/32 bytes, unit
 * (lg, c) = tokens [4lg, 4lg+4) x channels [8c, 8c+8) with the code of token u,
 * channel nt at bit (2*nt + u/2)*2*vb + (u%2)*vb -- a lossless permutation of
 * the same bits that lets one MFMA lane load its operand with one access.
 * kcodes rows are head_dim*key_bits/8 bytes.  4-bit keys use the reference's
 * pack as above; 3- and 2-bit keys (uniform) a permutation of it: each row is
 * head_dim/32 chunks of 32 channels (4*key_bits bytes each), and in chunk c the
 * little-endian field i (2*key_bits bits at bit 2*key_bits*i) holds
 * code(32c + 2i) | code(32c + 2i + 1) << key_bits, so one MFMA lane loads its
 * 32 channels with one access and reads a channel pair with one field.
 */
#ifndef TQK_H_
#define TQK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQK_OK 0
#define TQK_EINVAL 1        /* bad argument / shape (Python: ValueError) */
#define TQK_EUNSUPPORTED 2  /* configuration has no GPU form (Python: NotImplementedError) */
#define TQK_EHIP 3          /* a HIP runtime call failed (Python: RuntimeError) */
#define TQK_EWORKSPACE 4    /* workspace too small */

typedef struct tqk_cache_desc {
  int32_t n_kv_heads;           /* Hkv */
  int32_t n_q_heads;            /* Hq, a multiple of Hkv (q-head i reads kv-head i / (Hq/Hkv)) */
  int32_t head_dim;             /* D: 64, 128 or 256 (the MFMA decode serves 128; 64 and 256 run
                                   the VALU decode) */
  int32_t hot_window;           /* W; groups flush when the hot window exceeds W */
  int32_t group_tokens;         /* G = (W + 1) / 2, 1..256 */
  int32_t page_tokens;          /* P, divides G */
  int32_t key_bits;             /* 4 (asym-NF4 or uniform, see key_grid); 3 or 2 (uniform only) */
  int32_t value_bits;           /* 2, 3 or 4 (PolarQuant) */
  int32_t outliers_per_channel; /* k = max(1, round(G * outlier_frac)), 0 = no side-list */
  int32_t outlier_cap;          /* oent capacity per (group slot, head) */
  int32_t max_pages_per_seq;    /* block_table row stride */
  int32_t max_groups_per_seq;   /* group_table row stride */
  int32_t hot_ring;             /* ring capacity in tokens, >= W */
  int32_t n_pages;              /* physical pages in the pool (block_table entries index them) */
  float sm_scale;               /* softmax scale, 1/sqrt(D) */
  int32_t key_grid;             /* 0: asym-NF4 (gmean = the zero point, gscale = abs-max of the
                                   channel centred on it, levels NF4); 1: uniform (gmean = channel min,
                                   gscale = max(max - min, 1e-8) / (2^key_bits - 1), levels 0..2^key_bits-1);
                                   2: PolarQuant keys (TurboQuantKV with kind="key": the value
                                   encode on the keys, key_bits == value_bits, levels vcent, per-token
                                   norms in knorm; gscale 1, gmean 0, no side-list) */
  int32_t zero_point;           /* asym-NF4 zero point (turboquant_pro/per_channel_kv.py:327-345):
                                   0 "calibrated", the channel mean over the group;
                                   1 "sparse", the channel mean on the dc_mask channels, 0 elsewhere;
                                   2 "bias", zp_mean[g] of the group's index g (host-computed) */
  int32_t input_f32;            /* 0: keys, values and queries arrive as fp16 (the hot ring is fp16);
                                   1: as fp32 (an fp32 hot ring; codes from the fp32 values, bit-exact
                                   to the reference on fp32 input, true codes kept at side-list
                                   positions; decoded by the VALU kernel) */
  uint32_t dc_mask[8];          /* sparse: channel j is a DC channel when bit j % 32 of word j / 32 is set */
} tqk_cache_desc;

typedef struct tqk_cache_ptrs {
  uint8_t* kcodes;
  uint8_t* vcodes;
  float* vnorm;
  float* gscale;
  float* gmean;
  int32_t* ocount;
  uint32_t* oent;
  void* hot_k;          /* fp16, or fp32 when input_f32 */
  void* hot_v;
  const int32_t* block_table;
  const int32_t* group_table;
  const float* pi;      /* (D, D) row-major: unrotate y -> y @ pi */
  const float* pi_t;    /* (D, D) row-major: rotate x -> x @ pi_t */
  const float* vcent;   /* 2^vb fp32 value centroids (already / sqrt(D)) */
  const float* vbnd;    /* 2^vb - 1 fp32 value boundaries */
  const float* zp_mean; /* zero_point 2: [max_groups_per_seq][n_kv_heads][head_dim] zero points of
                           the groups starting at token g * group_tokens; unused otherwise */
  float* knorm;         /* key_grid 2: [n_kv_heads][n_pages][page_tokens] f32 key norms; unused otherwise */
} tqk_cache_ptrs;

/* Library ABI version (bumped on any signature or layout change); this header is version 9. */
int tqk_version(void);

/* Validate a descriptor; TQK_OK when the GPU path supports it. */
int tqk_check_desc(const tqk_cache_desc* d);

/* Bytes of decode workspace needed for `batch` sequences of at most
 * `max_len` tokens (0 when batch > n_pages: a decode call takes at most
 * n_pages sequences).  Host function, no GPU work.  The workspace starts with
 * the arrival counters of tqk_decode's in-kernel merge, one 32-bit word per
 * (sequence, kv head) for n_pages sequences -- a region that depends on the
 * descriptor only, so it never moves between calls -- then holds the split
 * partials: zero-fill a new workspace once before its first tqk_decode; every
 * completed call leaves the counters at zero again, whatever the batch and
 * max_len of the next call.  Calls that share a workspace must not overlap. */
size_t tqk_decode_workspace_bytes(const tqk_cache_desc* d, int32_t batch, int32_t max_len);

/*
 * Fused decode-step attention over the two-tier cache, one query token per
 * sequence: out[b][i] = softmax(q[b][i] . K_b^T * sm_scale) V_b over all
 * seq_lens[b] cached tokens of kv-head i / (Hq/Hkv), with the coded groups
 * attended in code space (no reconstruction) and the hot window in fp16.
 *   q        [batch][n_q_heads][head_dim] fp16 (fp32 when input_f32)
 *   seq_lens [batch] i32 (device), every entry in [1, max_len]
 *   out      [batch][n_q_heads][head_dim] fp32
 * Replaces TurboQuantKVCache.fused_decode (turboquant_pro/core.py:1168-1265)
 * and the per-page kernel launches behind it (turboquant_pro/kv_kernel.py:319-381).
 */
int tqk_decode(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
               const void* q, const int32_t* seq_lens, int32_t max_len, float* out,
               void* workspace, size_t workspace_bytes, void* stream);

/*
 * tqk_decode without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The split
 * partials and arrival counters live in the library's own device scratch
 * array, 32 MiB per GPU, held until the process ends; the call allocates
 * nothing.  Limits: batch * n_kv_heads <= 65536, and the partials
 * (batch * n_q_heads * splits * (head_dim + 2) floats, the part of
 * tqk_decode_workspace_bytes after the counters) must fit the rest of the
 * 32 MiB; otherwise TQK_EWORKSPACE.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other threads) race.
 * The first call on a device resolves the array's address and zeroes its
 * counters on `stream`.
 */
int tqk_decode_noalloc(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                       const void* q, const int32_t* seq_lens, int32_t max_len, float* out,
                       void* stream);

/*
 * Same step, returning the unnormalised online-softmax state instead of the
 * output: m [batch][n_q_heads], l [batch][n_q_heads], acc [batch][n_q_heads][D]
 * (real space), so that out = acc / l and states merge with
 * merge_partials (turboquant_pro/kv_fused.py:139-153; the kernel-level
 * partial contract of turboquant_pro/kv_kernel.py:212-213).
 */
int tqk_decode_partials(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                        const void* q, const int32_t* seq_lens, int32_t max_len,
                        float* m, float* l, float* acc, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * The two phases of tqk_decode, for callers that time or overlap them:
 * tqk_decode_splits writes every split's online-softmax state into the
 * workspace; tqk_decode_merge combines them (the flash-combine of
 * turboquant_pro/kv_kernel.py:377-381), rotates the coded part back and
 * normalises.  Same arguments and workspace as tqk_decode.
 */
int tqk_decode_splits(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                      const void* q, const int32_t* seq_lens, int32_t max_len,
                      void* workspace, size_t workspace_bytes, void* stream);
int tqk_decode_merge(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                     int32_t max_len, float* out, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Quantize-on-flush: encode `n_items` groups, item i = (items[2i], items[2i+1])
 * = (sequence b, group index g), all kv heads.  Token t of sequence b is read
 * from the hot ring when t < prev_len[b], else from the appended chunk at
 * chunk_k[b][h][t - prev_len[b]][:] (chunk row stride chunk_tokens).
 * Writes K/V codes, norms, group scale/mean and the outlier side-list
 * bit-exactly as PerChannelKV.compress (turboquant_pro/per_channel_kv.py:285-401)
 * and TurboQuantKV.compress (turboquant_pro/core.py:542-617) would.
 * `overflow` (device i32, caller zeroes it) gets bit 0 when a (group, head)
 * has more outliers than outlier_cap (the side-list is then truncated) and
 * bit 1 when a value vector's norm exceeds 16376 (the decode keeps softmax
 * weights <= 4 and carries weight * norm in fp16, whose largest value is
 * 65504: such a cache cannot be decoded).
 * Replaces TurboQuantKVCache._flush_to_cold (turboquant_pro/core.py:1011-1038).
 */
int tqk_encode_groups(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                      int32_t n_items, const int32_t* items, const int32_t* prev_len,
                      const void* chunk_k, const void* chunk_v, int32_t chunk_tokens,
                      int32_t* overflow, void* stream);

/*
 * Copy appended tokens into the hot ring: for each sequence b, tokens
 * [max(prev_len[b], hot_start[b]), prev_len[b] + n_new[b]) of the chunk go to
 * ring slot t % hot_ring.  Part of TurboQuantKVCache.append
 * (turboquant_pro/core.py:986-1009).
 */
int tqk_append_hot(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t batch,
                   const int32_t* prev_len, const int32_t* n_new, const int32_t* hot_start,
                   const void* chunk_k, const void* chunk_v, int32_t chunk_tokens,
                   void* stream);

/*
 * Reconstruct fp32 keys and values of `n_items` groups (items as in
 * tqk_encode_groups): kout/vout [n_items][n_kv_heads][G][D].  The GPU form of
 * PerChannelKV.decompress (turboquant_pro/per_channel_kv.py:497-539) and
 * TurboQuantKV.decompress (turboquant_pro/core.py:619-654), used by
 * TurboQuantKVCache.get_keys / get_values.
 */
int tqk_dequant_groups(const tqk_cache_desc* d, const tqk_cache_ptrs* p, int32_t n_items,
                       const int32_t* items, float* kout, float* vout, void* stream);

/*
 * Stateless block quantizers: one (B, H, S, D) block, every (b, h) pair one
 * quantization group of S tokens (any S >= 1), fp16 or fp32 input, outputs in
 * the reference containers' layouts.  The plugin / block-store path
 * (PerChannelKV.compress on whole layer blocks, turboquant_pro/connectors/
 * vllm_v1.py:298-322).
 */
typedef struct tqk_block_desc {
  int32_t batch;                /* B */
  int32_t n_heads;              /* H */
  int32_t tokens;               /* S >= 1 */
  int32_t head_dim;             /* D: 64, 128 or 256 */
  int32_t bits;                 /* keys: 4, 3 or 2 (3 and 2 uniform only); values: 2, 3 or 4 */
  int32_t key_grid;             /* keys: 0 asym-NF4, 1 uniform */
  int32_t zero_point;           /* asym-NF4 keys: 0 calibrated, 1 sparse, 2 given (zp), as in tqk_cache_desc */
  int32_t outliers_per_channel; /* keys: k = max(1, round(S * outlier_frac)), 0 = no side-list */
  int32_t outlier_cap;          /* keys: side-list capacity per (b, h) */
  int32_t input_f32;            /* 1: x is fp32, 0: x is fp16 */
  uint32_t dc_mask[8];          /* sparse: DC channels, as in tqk_cache_desc */
} tqk_block_desc;

/*
 * Per-channel key quantization of x [B][H][S][D] (PerChannelKV.compress,
 * turboquant_pro/per_channel_kv.py:269-401): packed [B*H*S*D*bits/8] u8 (the
 * reference's packed indices, true codes at outlier positions), scale and
 * zero [B][H][D] f32 (asym-NF4: nf4_scale and the zero point; uniform: scale
 * and channel min), the side-list of each (b, h) in (s, j) order as
 * out_pos [B*H][outlier_cap] u32 (s * D + j) and out_val [B*H][outlier_cap]
 * fp16, and out_count [B*H] i32 (may exceed outlier_cap: the list is then
 * truncated).  zp [H][D] f32 for zero_point 2, else unused.
 */
int tqk_encode_key_block(const tqk_block_desc* d, const void* x, const float* zp, uint8_t* packed,
                         float* scale, float* zero, uint32_t* out_pos, uint16_t* out_val,
                         int32_t* out_count, void* stream);

/*
 * PolarQuant of x [B][H][S][D] (TurboQuantKV.compress(kind="value"),
 * turboquant_pro/core.py:542-617): packed [B*H*S][D*bits/8] u8 (the
 * reference's little-endian bit stream per token) and norms [B*H*S] f32.
 * pi is the cache's (D, D) row-major Pi (rotation y_e = sum_d u_d * pi[e][d],
 * i.e. u @ pi_t), vbnd the 2^bits - 1 boundaries.
 */
int tqk_encode_value_block(const tqk_block_desc* d, const void* x, const float* pi,
                           const float* vbnd, uint8_t* packed, float* norms, void* stream);

/*
 * Key reconstruction (PerChannelKV.decompress, turboquant_pro/per_channel_kv.py:
 * 497-539): out [B][H][S][D] f32 = zero + scale * level[code] (level NF4 or
 * the code itself for key_grid 1), then out[out_idx[i]] = fp32(out_val[i])
 * for the n_out flat indices of the reference's side-list (an index outside
 * [0, B*H*S*D) is skipped; callers validate the list beforehand).
 */
int tqk_dequant_key_block(const tqk_block_desc* d, const uint8_t* packed, const float* scale,
                          const float* zero, int32_t n_out, const int32_t* out_idx,
                          const uint16_t* out_val, float* out, void* stream);

/*
 * Value reconstruction (TurboQuantKV.decompress, turboquant_pro/core.py:
 * 619-654): out [B][H][S][D] f32 = (vcent[code] @ pi) * norm per token.
 */
int tqk_dequant_value_block(const tqk_block_desc* d, const uint8_t* packed, const float* norms,
                            const float* pi, const float* vcent, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TQK_H_ */
