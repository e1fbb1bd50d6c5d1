/*
 * rec_amd — C ABI of the MI355X (gfx950) quantized-KV attention library.
 *
 * Every pointer is a caller-owned device buffer unless stated otherwise; the
 * library allocates nothing.  Calls are asynchronous on `stream` (a
 * hipStream_t, NULL for the default stream) and return 0 on success or a
 * negative REC_E* code, with a message for the calling thread available from
 * rec_last_error().  Nothing throws across this boundary.
 *
 * Cache layout per layer, in 32-token blocks (bh = b*Hkv + h, C = capacity, a
 * multiple of 32, head_dim D = 128, scales and zero-points are IEEE fp16 bit
 * patterns; token t of a block sits at position p = 8*((t>>2)&3) + 4*(t>>4) + (t&3)):
 *   int8 K codes  int8  [B][Hkv][C/32][2][32][64]   half m = dims 64m..64m+63, row = token t
 *   int4 K codes  uint8 [B][Hkv][C/32][32][4][2][8]  row = token t, [byte run r][half m][8 bytes]:
 *                                                   byte 8r+i of half m holds dims 64m+16r+2i, +1 (low nibble even)
 *   int8 V codes  int8  [B][Hkv][C/32][4][16][4][2][8]  dim 16n+c, position p = 8g+e at
 *                                                   [n/2][c][g][n%2][e]
 *   int4 V codes  uint8 [B][Hkv][C/32][2][16][4][4][4]  dim 16n+c, position p = 8g+e at
 *                                                   [n/4][c][g][n%4][e/2], low nibble = even e
 *   int8 scales   fp16  [B][Hkv][C/32][32]          one per (token, head), position p
 *   int4 scale/zp fp16  [B][Hkv][C/32][4][32]       per 32-dim group, at slot
 *                                                    (p & ~7) | 2*(p & 3) | ((p >> 2) & 1)
 * Quantizers: int8 symmetric s = fp16(amax/127), q = clamp(rint(x/s), ±127);
 * uint4 asymmetric over [min(0, x), max(0, x)], s = fp16(range/15),
 * z = clamp(rint(-min/s), 0, 15), q = clamp(rint(x/s) + z, 0, 15).
 *
 * MLX-style affine format (k_bits = REC_AFFINE8 with v_bits = REC_AFFINE4; the
 * reference's MixedQuantizedKVCache, engine/src/rec_mlx/model.py:40-82, group
 * 64): x = s*q + b with bf16 scale s and bias b per (token, 64-dim group).
 * Key codes are uint8 in the int8 K layout, value codes uint4 in the int4 V
 * layout; each "scales" buffer holds bf16 [B][Hkv][C/32][2 (scale, bias)][2
 * groups][32] at the int4 slot order; the zeros pointers are unused (NULL).
 * Quantizer: MLX's affine_quantize (w_max = max(0, max w), w_min = min w,
 * step (w_max - w_min)/n_bins, the larger-magnitude extreme made exact, codes
 * round-half-away((w - b)/s) clamped to [0, n_bins]), scale and bias rounded to
 * bf16.  REC_AFFINE8_F16 with REC_AFFINE4_F16 is the same format with fp16
 * scales and biases (rounded to nearest even): the reference allocates them in
 * the keys' dtype (model.py:57-58), fp16 for an fp16 model.
 */
#ifndef REC_AMD_H
#define REC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  REC_OK = 0,
  REC_EINVAL = -1,       /* bad shape, dtype or argument */
  REC_EALIGN = -2,       /* a buffer is not 16-byte aligned */
  REC_ECAPACITY = -3,    /* tokens beyond the cache capacity */
  REC_EWORKSPACE = -4,   /* workspace missing or too small */
  REC_ELAUNCH = -5,      /* the HIP runtime rejected a launch */
  REC_EUNSUPPORTED = -6  /* a valid request this library does not implement */
};

/* Element types of the float inputs (queries, new keys/values). */
enum { REC_F16 = 0, REC_BF16 = 1, REC_F32 = 2 };

/* k_bits / v_bits: 8 (int8 symmetric), 4 (uint4 group 32), or an affine pair
 * (bf16 or fp16 scales and biases) */
enum { REC_AFFINE8 = 0x108, REC_AFFINE4 = 0x104, REC_AFFINE8_F16 = 0x208, REC_AFFINE4_F16 = 0x204 };

/* Library version, e.g. "rec_amd 0.1.0 gfx950". */
const char* rec_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* rec_last_error(void);

/*
 * Quantize-on-append: quantize rows [0, L) of k_new / v_new (B, Hkv, L, D),
 * element strides (sb, sh, st) with unit dim stride, and store them at cache
 * positions [offset, offset + L).  k_bits / v_bits are 8 or 4; zeros are used
 * (and required) for 4-bit only.
 * Replaces the quantize-and-write step of MixedQuantizedKVCache.update_and_fetch,
 * engine/src/rec_mlx/model.py:76-81 (mx.quantize at :77-78, slice writes at :79-81).
 */
int rec_kv_append(const void* k_new, const void* v_new, int in_dtype,
                  int64_t k_sb, int64_t k_sh, int64_t k_st,
                  int64_t v_sb, int64_t v_sh, int64_t v_st,
                  int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros,
                  int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros,
                  int B, int Hkv, int L, int D, int64_t offset, int64_t capacity, void* stream);

/* Split count the library would pick for a decode over T tokens. */
int rec_decode_default_splits(int B, int Hkv, int64_t T);

/*
 * Bytes of workspace a decode call with `splits` requested splits needs, for
 * every entry point (a fused append launches at most max(splits, 2) splits;
 * splits <= 0: the largest plan).
 */
size_t rec_decode_workspace_bytes(int B, int Hkv, int splits);

/*
 * Zero a workspace with a kernel (capturable in a HIP graph).  Decode calls
 * need no particular workspace contents; this is for callers that want a
 * deterministic buffer.  One workspace serves one stream at a time.
 */
int rec_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/*
 * GQA decode attention over the first T cached tokens for one query token per
 * sequence: q (B, Hq, D) with element strides (q_sb, q_sh), q-head h reads
 * kv-head h / (Hq/Hkv), Hq/Hkv <= 8; q rows start 16-byte aligned with strides
 * that are multiples of 4 elements (else REC_EALIGN).  scores = scale * q·k̂; `sinks` (Hq fp32
 * logits, or NULL) join the softmax denominator; out (B, Hq, D), 16-byte
 * aligned, of out_dtype: REC_F32, or REC_BF16 / REC_F16 (the fp32 result
 * rounded to nearest even, the query dtype the reference returns,
 * model.py:132-139 — no separate cast launch).
 * bias (NULL: none): an additive score bias, the reference's mask array
 * (model.py:122-128) after its broadcasting — a bool mask as 0 / -inf, a float
 * mask as it is, in natural-log units like the scores — with element
 * (b, kv head h, group member g, key t) at bias[b*bias_sb + h*bias_skv +
 * g*bias_sg + t] (strides 0 where the mask broadcasts, non-negative
 * multiples of 4; 16-byte aligned; bias_extent = elements readable from
 * bias, below 2^29).  A row that every key leaves out gets the sink alone
 * (zeros without sinks).
 * splits <= 0 picks rec_decode_default_splits().
 * Replaces quantized_attention_with_sinks, engine/src/rec_mlx/model.py:108-139
 * (split-K structure of engine/src/rec_mlx/kernels/megakernel.py:619-693 and
 * merge :276-318).
 */
int rec_decode_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                    int k_bits, const void* k_codes, const uint16_t* k_scales, const uint16_t* k_zeros,
                    int v_bits, const void* v_codes, const uint16_t* v_scales, const uint16_t* v_zeros,
                    const float* sinks, float scale,
                    const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_extent,
                    int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                    void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * One decode step: quantize-append the single new token k_new / v_new
 * (B, Hkv, 1, D) at cache position T-1 and attend over all T tokens, the new
 * one included, in one attention launch (plus the split merge), as
 * Attention.__call__ does
 * (engine/src/rec_mlx/model.py:177-190: update_and_fetch, then
 * quantized_attention_with_sinks).
 */
int rec_decode_append_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                           const void* k_new, const void* v_new, int new_dtype,
                           int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                           int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros,
                           int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros,
                           const float* sinks, float scale,
                           int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                           void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * rec_decode_append_attn for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * same arguments without a workspace, the same kernels, and the split
 * partials kept in a static device array of rec_decode_scratch_bytes() bytes
 * (8 MiB, one per GPU, held until the process ends).  No allocation of any
 * kind.  A plan whose partials exceed it (B * Hkv * splits above about 2,000)
 * returns REC_EWORKSPACE before anything is launched.  Every call on one GPU
 * shares that GPU's array: calls that may overlap (on different streams)
 * race and must be ordered by the caller.  No counterpart in the reference.
 */
int rec_decode_append_attn_noalloc(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                                   const void* k_new, const void* v_new, int new_dtype,
                                   int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                                   int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros,
                                   int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros,
                                   const float* sinks, float scale,
                                   int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                                   int out_dtype, void* out, void* stream);
size_t rec_decode_scratch_bytes(void);

/*
 * The two launches of a decode step, for callers that schedule them apart
 * (for instance to time or overlap them).  rec_decode_partial takes the
 * arguments of rec_decode_append_attn; k_new/v_new NULL means no append.  It
 * writes `out` directly when the request resolves to a single split, else the
 * split partials into the workspace.  rec_decode_merge then combines those
 * partials into `out` (nothing to do for a single split); it must be given the
 * B, Hq, Hkv, T, splits, sinks and workspace of the partial call, and
 * appended = 1 if that call appended a token.
 * Together they are rec_decode_append_attn: the split-K partial of
 * engine/src/rec_mlx/kernels/megakernel.py:619-693 and its merge :276-318.
 */
int rec_decode_partial(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                       const void* k_new, const void* v_new, int new_dtype,
                       int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                       int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros,
                       int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros,
                       const float* sinks, float scale,
                       int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                       void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

int rec_decode_merge(const float* sinks, int B, int Hq, int Hkv, int64_t T, int splits, int appended,
                     void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * Chunked prefill: the last L of the T cached tokens are new (already
 * quantize-appended with rec_kv_append); their queries q (B, Hq, L, D), element
 * strides (q_sb, q_sh, q_st), bf16 or f16 (float32 queries: one
 * rec_decode_attn per query row i over the first T-L+i+1 tokens under a
 * causal mask, as the Python layer does), attend over all T tokens — with
 * causal != 0, query i sees tokens [0, T-L+i]; window > 0 further limits
 * query position p to keys > p - window (a sliding-window mask array of
 * model.py:122-128; window 0 = none) — with optional sink logits.
 * out (B, Hq, L, D) of out_dtype (REC_F32, REC_BF16 or REC_F16, as the decode).
 * bias: as rec_decode_attn's, with query l of the chunk at + l*bias_sl; with a
 * bias, causal and window must be 0 (the bias carries the whole mask) and the
 * chunk takes the tiled kernel.  Any cache format of rec_decode_attn (int8 or uint4
 * in any mix, or an affine pair): K/V tiles are dequantized into on-chip
 * memory, never to HBM — int8 codes exactly with the row scales applied to
 * scores and probabilities, 4-bit and affine values as x̂ rounded to the
 * query dtype, as the reference dequantizes before its attention.  A chunk
 * of at most 32 (query, head) rows per KV head (64 over a cache of 16,384
 * tokens or more) over any of these caches (no window, no bias) streams the
 * cache through registers instead, as the decode does, with the same values;
 * its splits and workspace are the same.
 * splits: key splits (<= 0: automatic, 1: none, at most 64).  A short chunk
 * over a long cache (few query blocks x KV heads x batch) splits the keys so
 * that the launch fills the chip; the partials go to `workspace`
 * (rec_prefill_workspace_bytes) and a second kernel merges them.  An automatic
 * plan without a workspace (NULL or too small) runs unsplit; an explicit
 * split count > 1 without one fails with REC_EWORKSPACE.
 * Replaces the prefill branch of Attention.__call__,
 * engine/src/rec_mlx/model.py:191-203 (mask rule :122-125).
 */
int rec_prefill_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                     int k_bits, const void* k_codes, const uint16_t* k_scales, const uint16_t* k_zeros,
                     int v_bits, const void* v_codes, const uint16_t* v_scales, const uint16_t* v_zeros,
                     const float* sinks, float scale, int causal, int window,
                     const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_sl,
                     int64_t bias_extent,
                     int B, int Hq, int Hkv, int D, int L, int64_t T, int64_t capacity,
                     int splits, void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/* Workspace bytes a prefill launch of L queries with Hq query and Hkv KV heads
 * needs for `splits` key splits (<= 0: the most the automatic plan can use);
 * 0 when it does not split (or for an invalid shape).
 * Serves rec_prefill_attn and rec_prefill_bf16; no counterpart in the
 * reference, whose prefill is one library call. */
size_t rec_prefill_workspace_bytes(int B, int Hq, int Hkv, int L, int splits);

/*
 * bf16 KV cache (the reference's production format): K and V are (B, Hkv,
 * capacity, 128) bf16 tensors with unit dim stride, token stride 128 and
 * element strides (sb, sh) for batch and head — the [2][Hkv][cap][128] layer
 * region of KVStorage (engine/src/rec_mlx/cache.py:48-95) is K = region[0],
 * V = region[1].  Storage must be 16-byte aligned, strides multiples of 8.
 *
 * rec_kv_write_bf16: store rows [0, L) of k_new / v_new (any float dtype,
 * rounded to bf16) at positions [offset, offset + L).
 * Replaces KVStorage.write and its flint_write_kv kernel,
 * engine/src/rec_mlx/cache.py:30-45, :97-119.
 */
int rec_kv_write_bf16(const void* k_new, const void* v_new, int in_dtype,
                      int64_t k_sb, int64_t k_sh, int64_t k_st,
                      int64_t v_sb, int64_t v_sh, int64_t v_st,
                      void* k, int64_t kc_sb, int64_t kc_sh, void* v, int64_t vc_sb, int64_t vc_sh,
                      int B, int Hkv, int L, int D, int64_t offset, int64_t capacity, void* stream);

/*
 * rec_ring_join_bf16: the keys and values a chunk attends over in a
 * sliding-window ring, in one launch — the n_held tokens in sequence order
 * (token i at ring slot (head + i) mod capacity; the ring is (B, Hkv,
 * capacity, 128) bf16 with element strides (r*_sb, r*_sh), token stride 128)
 * followed by rows [0, L) of k_new / v_new (any float dtype, rounded to
 * bf16), into contiguous (B, Hkv, n_held + L, 128) bf16 k_out / v_out.
 * place != 0: the chunk's last min(L, capacity) rows (sequence positions
 * offset + j) also go to their slots (offset + j) mod capacity, each held
 * token read before its slot is rewritten — the whole update of the ring.
 * Replaces the concatenation of the held window and the chunk, and the
 * ring's rewrite, in FixedSlidingKVCache.update_and_fetch,
 * engine/src/rec_mlx/cache.py:227-247.
 */
int rec_ring_join_bf16(void* k_ring, void* v_ring, int64_t rk_sb, int64_t rk_sh,
                       int64_t rv_sb, int64_t rv_sh, int64_t capacity, int64_t head, int64_t n_held,
                       int64_t offset, int place, const void* k_new, const void* v_new, int in_dtype,
                       int64_t k_sb, int64_t k_sh, int64_t k_st,
                       int64_t v_sb, int64_t v_sh, int64_t v_st,
                       void* k_out, void* v_out, int B, int Hkv, int L, int D, void* stream);

/*
 * GQA decode attention over the first T tokens of a bf16 K/V cache, with an
 * optional fused write of the newest token (k_new / v_new (B, Hkv, 1, D), any
 * float dtype, stored at position T-1 first; NULL: no write).  Query, sinks,
 * scale, bias, splits, workspace and output as rec_decode_attn; the split-K
 * partial and the merge are both launched.
 * Replaces the attention of Attention.__call__ over a FixedKVCache,
 * engine/src/rec_mlx/model.py:204-211 (FixedKVCache.update_and_fetch first,
 * cache.py:145-150), whose fused-decoder form is the bf16 split-K partial of
 * engine/src/rec_mlx/kernels/megakernel.py:619-693 and merge :276-318.
 */
int rec_decode_bf16(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                    const void* k_new, const void* v_new, int new_dtype,
                    int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh,
                    void* k, int64_t k_sb, int64_t k_sh, void* v, int64_t v_sb, int64_t v_sh,
                    const float* sinks, float scale,
                    const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_extent,
                    int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                    void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * rec_decode_bf16_ring: one decode step of a sliding-window ring (token p of
 * the sequence in slot p mod capacity): the new token (k_new / v_new, both
 * required) is written into `slot` and the query attends over the T
 * occupied slots — softmax is order-free, so the slots are read as they lie.
 * Arguments otherwise as rec_decode_bf16; 0 <= slot < T.
 * Replaces FixedSlidingKVCache.update_and_fetch of one token and the
 * attention over it, engine/src/rec_mlx/cache.py:227-247 and
 * engine/src/rec_mlx/model.py:204-211.
 */
int rec_decode_bf16_ring(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                         const void* k_new, const void* v_new, int new_dtype,
                         int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh,
                         void* k, int64_t k_sb, int64_t k_sh, void* v, int64_t v_sb, int64_t v_sh,
                         const float* sinks, float scale, int B, int Hq, int Hkv, int D, int64_t T,
                         int64_t capacity, int64_t slot, int splits, void* workspace,
                         size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * Dequantize cache rows [0, T) of any format (k_bits / v_bits as rec_kv_append)
 * into bf16 K and V tensors (B, Hkv, T, 128), contiguous and 16-byte aligned:
 * x̂ formed in float32 (int8 q*s, uint4 (q - z)*s, affine q*s + b), rounded to
 * bf16.  Replaces the dequantization of the prefill branch,
 * engine/src/rec_mlx/model.py:194-195 (the attention then runs on the bf16
 * tensors, rec_prefill_bf16).
 */
int rec_kv_dequant_bf16(int k_bits, const void* k_codes, const uint16_t* k_scales, const uint16_t* k_zeros,
                        int v_bits, const void* v_codes, const uint16_t* v_scales, const uint16_t* v_zeros,
                        int B, int Hkv, int64_t T, int64_t capacity, void* k_out, void* v_out, void* stream);

/*
 * Prefill attention over a bf16 K/V cache (the FixedKVCache / FixedSlidingKVCache
 * path): the L queries (B, Hq, L, D) bf16 or f16, element strides q_sb/q_sh/q_st,
 * are the newest L of the T cached tokens (query i at position T-L+i); K and V
 * are (B, Hkv, >=T, 128) bf16 with token stride 128 and 16-byte aligned rows.
 * causal: query p sees keys <= p; window > 0 further limits it to keys
 * > p - window (the sliding-window mask of cache.py:199-205).  Sinks, scale and
 * the fp32 output (B, Hq, L, 128), splits and workspace as rec_prefill_attn.
 * Replaces mx.fast.scaled_dot_product_attention over a FixedKVCache or
 * FixedSlidingKVCache in Attention.__call__, engine/src/rec_mlx/model.py:204-211
 * (the 512-query windowed form: engine/src/rec_mlx/m4_max_prefill.py:86-104).
 */
int rec_prefill_bf16(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                     const void* k, int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh,
                     const float* sinks, float scale, int causal, int window,
                     const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_sl,
                     int64_t bias_extent,
                     int B, int Hq, int Hkv, int D, int L, int64_t T, int splits,
                     void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream);

/*
 * A plain streaming read of `bytes` (a positive multiple of 16) at p (16-byte
 * aligned) by `workgroups` workgroups of 256 threads; `out` (workgroups
 * uint32, device memory) is written only in the rare case the XOR of the
 * data hits a fixed value.  No counterpart in the reference: the one-launch
 * read floor of this part, against which the decode kernels are measured.
 */
int rec_stream_read(const void* p, int64_t bytes, int workgroups, uint32_t* out, void* stream);

/*
 * Growable bf16 layer region (KVStorage's banks): reserves the address range
 * of `rows` rows (B * 2 * Hkv for a layer: K then V per batch row) of
 * `max_tokens` tokens of `token_bytes` each, row r at base + r * max_tokens *
 * token_bytes, and maps device memory into it one bank of `bank_tokens`
 * tokens per row at a time.  Mapped banks never move, so growing copies
 * nothing and the region is one strided tensor (token stride token_bytes,
 * row stride max_tokens * token_bytes) for rec_kv_write_bf16,
 * rec_decode_bf16 and rec_prefill_bf16.  New banks hold undefined bytes.
 * rec_region_create: device ordinal; bank_tokens * token_bytes must be a
 * multiple of the device's mapping granularity (2 MiB on MI355X); *handle
 * and *base receive the region and its device address (nothing mapped yet).
 * rec_region_grow: map banks until `tokens` tokens per row are backed;
 * *capacity (may be NULL) receives the tokens now backed.
 * rec_region_destroy: unmap and free; no work on the region may be in flight.
 * Replaces the bank list of KVStorage, engine/src/rec_mlx/cache.py:46-84
 * (four 65,536-token banks added without copying, the kernel picking a bank
 * per token, engine/src/rec_mlx/kernels/megakernel.py:115-135).
 */
int rec_region_create(int device, int64_t rows, int64_t max_tokens, int64_t token_bytes, int64_t bank_tokens,
                      void** handle, void** base);
int rec_region_grow(void* handle, int64_t tokens, int64_t* capacity);
int rec_region_destroy(void* handle);

/*
 * int4 group-64 GEMV (MLX affine 4-bit, the format of the decoder's
 * projections, experts and lm head): y[m] = x[m] · Wᵀ for an (N, K) matrix
 * given as MLX words w (N, K/8) uint32 (code e of a word at bits 4e), bf16
 * scales and biases (N, K/64), element (r, k) = s·q + b.
 *
 * rec_q4_packed_bytes: bytes of the repacked matrix (0 if N < 1 or K is not a
 * positive multiple of 128).  Row tiles are 16 rows: the rows [16t, N) of a
 * packed matrix start at byte t · (K/128) · 1152.
 * rec_q4_pack: repack w / scales / biases (contiguous, 16-byte aligned w) into
 * `packed` (16-byte aligned, at least rec_q4_packed_bytes).  Once per matrix,
 * as the reference packs its weight banks, megakernel.py:1017-1040.
 * rec_q4_gemv: M (1..8) bf16 vectors x (row stride x_stride elements, a
 * multiple of 8; 16-byte aligned) to out (out_dtype REC_BF16, rounded to
 * nearest even as the reference stores bfloat16_t, or REC_F32; row stride
 * out_stride elements).  Matrices of one K stacked row-wise (their words,
 * scales and biases concatenated) pack as one, and one launch computes every
 * part, as the reference computes a layer's q, k and v heads in one pass
 * (megakernel.py:871-886).
 * Replaces q4 / dot16 (and q4_local) of
 * engine/src/rec_mlx/kernels/megakernel.py:161-232, the projections of
 * model.py:151-154 quantized by quantized.py:27-36 (group 64, 4 bits, affine).
 */
size_t rec_q4_packed_bytes(int64_t N, int64_t K);
int rec_q4_pack(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int64_t N, int64_t K,
                void* packed, size_t packed_bytes, void* stream);
int rec_q4_gemv(const void* packed, int64_t N, int64_t K, const uint16_t* x, int64_t x_stride, int M,
                void* out, int out_dtype, int64_t out_stride, void* stream);

/*
 * Many vectors (a prefill chunk's projections: the reference's
 * mx.quantized_matmul over L tokens, model.py:151-154, or q4 per token):
 * y[m] = x[m] · Wᵀ for M >= 1 bf16 vectors over the same packed matrix, as a
 * GEMM on matrix cores with rec_q4_gemv's arithmetic (codes and products
 * exact, sums in fp32).  x, x_stride, out, out_dtype and out_stride as
 * rec_q4_gemv; the workspace (16-byte aligned, at least
 * rec_q4_gemm_workspace_bytes(M, K)) receives x's group sums first.
 */
size_t rec_q4_gemm_workspace_bytes(int M, int64_t K);
int rec_q4_gemm(const void* packed, int64_t N, int64_t K, const uint16_t* x, int64_t x_stride, int M,
                void* out, int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REC_AMD_H */
