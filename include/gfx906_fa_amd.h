/* gfx906_fa_amd.h - C ABI of the MI355X (gfx950) Q8_0 paged-attention backend.
 *
 * Plain C: pointers, sizes and a hipStream_t.  No allocation, no
 * synchronisation: every entry point enqueues work on `stream` and returns a
 * hipError_t (hipErrorInvalidValue plus a line on stderr for an unsupported
 * configuration, otherwise the launch status).  Citations are to the
 * reference checkout (nick413-bit/gfx906-fa-vllm).
 *
 * Data formats
 * ------------
 * Q8_0 block: 32 int8 values plus one fp16 scale (kernel/ggml_shim.cuh:90-94).
 *   Quantization closed form (extension/gfx906_fa_quant.cu:51-84), per block:
 *     amax = max|x|; d = amax/127.f; id = d > 0 ? 1.f/d : 0;
 *     q = clamp(rintf(x*id), -128, 127); scale stored as fp16(d), RNE.
 *
 * AoS rows ("block_q8_0 rows"): a row of D values is D/32 blocks of 34 bytes,
 *   [fp16 d little-endian][32 x int8] each (extension/gfx906_fa_quant.cu:76-84).
 *
 * Planar page layout (this backend's KV cache, D = 128): the cache holds two
 *   planes (K, V).  A page of `block_size` tokens (a multiple of 16) of one
 *   kv-head in one plane is block_size/16 contiguous 2176-byte sub-pages, each
 *   covering 16 tokens:
 *     K sub-page: int8 q[t][d] at (b/2)*1024 + (4t+g)*16 + (b%2)*8 + d%8
 *                 (b = d/32, g = (d%32)/8),
 *                 fp16 scale[t][b] at 2048 + (4*t + b)*2
 *     V sub-page: int8 q[t][d] at (m/4)*1024 + ((t/4)*16 + d%16)*16 + (m%4)*4 + t%4
 *                 (m = d/16),
 *                 fp16 scale[t][b] at 2048 + ((t/4)*4 + b)*8 + (t%4)*2
 *   Address of (page p, kv-head h, sub-page j) in a plane:
 *     plane_base + p*cache_block_stride + h*cache_head_stride + j*2176.
 *   The values and scales are exactly the Q8_0 blocks of the AoS format;
 *   only their placement differs (chosen so the attention kernels load MFMA
 *   operands straight from HBM with aligned 16-byte loads).
 *
 * dtype codes: 0 = fp32, 1 = fp16, 2 = bf16.
 */
#ifndef GFX906_FA_AMD_H
#define GFX906_FA_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GFA_DTYPE_F32 = 0, GFA_DTYPE_F16 = 1, GFA_DTYPE_BF16 = 2 };

/* Library version string. */
const char *gfx906_fa_amd_version(void);

/* ---------------------------------------------------------------------------
 * (1) Dense Q8_0 quantize of contiguous fp16 rows [N, D] -> AoS rows
 *     [N, D/32*34].  Same name, arguments and semantics as the reference
 *     launcher (extension/gfx906_fa_quant.cu:206-223, declared at
 *     extension/gfx906_fa.cpp:38-44).
 */
hipError_t launch_quantize_q8_0_dense(const void *x, uint8_t *y, int N, int D,
                                      hipStream_t stream);

/* (1b) Same for fp16 / bf16 / fp32 input (x_dtype); N may exceed 2^31 rows
 *      of blocks.  No reference counterpart: the reference is fp16-only
 *      (extension/gfx906_fa.cpp:276). */
hipError_t gfx906_fa_amd_quantize_q8_0(const void *x, int x_dtype, uint8_t *y,
                                       int64_t N, int D, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (2) Quantize new key rows [T, Hkv, D] (element strides) and scatter them
 *     as AoS rows into a paged cache [NB, bs, Hkv, D/32*34] (byte strides) at
 *     slot_mapping[t] (int64; < 0 = skip).  All other bytes are untouched.
 *     Same name, arguments and semantics as the reference launcher
 *     (extension/gfx906_fa_quant.cu:225-253, declared at
 *     extension/gfx906_fa.cpp:46-60); key is fp16.
 */
hipError_t launch_reshape_and_cache_q8(const void *key, const int64_t *slot_mapping,
                                       uint8_t *k_cache_q8, int num_tokens,
                                       int num_kv_heads, int head_size, int block_size,
                                       int64_t key_token_stride, int64_t key_head_stride,
                                       int64_t cache_block_stride,
                                       int64_t cache_token_stride,
                                       int64_t cache_head_stride, hipStream_t stream);

/* (2b) Same with an input dtype (fp16 / bf16 / fp32). */
hipError_t gfx906_fa_amd_reshape_and_cache_q8(
    const void *key, int key_dtype, const int64_t *slot_mapping, uint8_t *k_cache_q8,
    int num_tokens, int num_kv_heads, int head_size, int block_size,
    int64_t key_token_stride, int64_t key_head_stride, int64_t cache_block_stride,
    int64_t cache_token_stride, int64_t cache_head_stride, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (3) Paged -> contiguous gather.  For s < num_seqs, h < Hkv, t < Sk:
 *       lb = t / block_size; pb = lb < max_blocks ? block_table[s][lb] : -1;
 *       if t < seq_lens[s] and pb >= 0: copy the K row (bytes_per_row bytes)
 *       and the V row (D fp16) of (pb, t % block_size, h);
 *       else zero the V row and leave the K row untouched.
 *     Outputs: k_out [B, Hkv, Sk, bytes_per_row], v_out [B, Hkv, Sk, D] fp16.
 *     K strides in bytes, V strides in fp16 elements.  Same name, arguments
 *     and semantics as the reference (extension/gfx906_fa_gather.cu:362-425,
 *     v2 contract at extension/gfx906_fa_gather.cu:190-357, declared at
 *     extension/gfx906_fa.cpp:94-115).
 */
hipError_t launch_gather_paged_kv_q8(
    const uint8_t *key_cache_q8, const void *value_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, void *v_out, int num_seqs, int num_kv_heads,
    int Sk, int D, int bytes_per_row, int block_size, int max_blocks_per_seq,
    int64_t cache_block_stride, int64_t cache_token_stride, int64_t cache_head_stride_q8,
    int64_t v_cache_block_stride, int64_t v_cache_token_stride,
    int64_t v_cache_head_stride, hipStream_t stream);

/* (3b) Same contract over generic row byte sizes (k_row_bytes, v_row_bytes;
 *      all strides in bytes), e.g. an AoS Q8_0 V cache (v_row_bytes = 136):
 *      the Q8/Q8 variant of (3). */
hipError_t gfx906_fa_amd_gather_rows(
    const uint8_t *k_cache, const uint8_t *v_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, uint8_t *v_out, int num_seqs,
    int num_kv_heads, int Sk, int k_row_bytes, int v_row_bytes, int block_size,
    int max_blocks_per_seq, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, int64_t v_block_stride, int64_t v_token_stride,
    int64_t v_head_stride, hipStream_t stream);

/* (3c) Gather from the planar K+V cache into AoS rows, same validity rule as
 *      (3): k_out, v_out [B, Hkv, Sk, 136]; invalid tokens get a zero V row
 *      and an untouched K row.  Replaces the reference's legacy torch gather
 *      (extension/gfx906_fa_paged.py:148-194) for this cache. */
hipError_t gfx906_fa_amd_gather_planar(
    const uint8_t *k_cache, const uint8_t *v_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, uint8_t *v_out, int num_seqs,
    int num_kv_heads, int Sk, int head_size, int block_size, int max_blocks_per_seq,
    int64_t cache_block_stride, int64_t cache_head_stride, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (4) Quantize-and-write K and V of new tokens into the planar cache.
 *     key/value [T, Hkv, D] (element strides, dtype fp16/bf16/fp32, D = 128),
 *     slot_mapping int64 [T] (< 0 = skip).  Replaces the reference's
 *     do_kv_cache_update pair (fp16 triton write + K-only Q8 side buffer,
 *     extension/gfx906_fa_backend.py:405-442; kernel
 *     extension/gfx906_fa_quant.cu:150-200): one launch, K and V both Q8_0.
 */
hipError_t gfx906_fa_amd_cache_write_kv(
    const void *key, const void *value, int dtype, const int64_t *slot_mapping,
    uint8_t *k_cache, uint8_t *v_cache, int num_tokens, int num_kv_heads, int head_size,
    int block_size, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, int64_t cache_block_stride,
    int64_t cache_head_stride, hipStream_t stream);

/* (4b) Fused rotary embedding + (4).  query [T, Hq, D] and key [T, Hkv, D]
 *      are rotated in place, then the rotated key and value are written as
 *      (4) does.  Rotary semantics (vLLM's rotary embedding): cos and sin are
 *      cos_sin_cache[positions[t]][0 .. rot_dim/2) and [rot_dim/2 .. rot_dim)
 *      (row stride cos_sin_stride elements, dtype cos_sin_dtype), converted
 *      to the model dtype; each pair (x, y) - (i, i + rot_dim/2) when
 *      is_neox, else (2i, 2i+1) - becomes (x*cos - y*sin, y*cos + x*sin)
 *      with every operation rounded to the model dtype; dims >= rot_dim are
 *      untouched.  Positions outside [0, max_position) leave their rows
 *      unrotated (nothing is read out of the cos/sin table).
 *      Requirements: fp16/bf16, D = 128, rot_dim <= 128 and a multiple of 16
 *      (neox) or 8, q/k/v rows 16-byte aligned (element strides multiples of
 *      8), cos/sin rows 8-byte aligned.
 *      Replaces the reference backend's declared absence of this fusion
 *      (fused_rope_kvcache_supported() returning False,
 *      extension/gfx906_fa_backend.py:444-445) for vLLM's fused
 *      rope + KV-cache-update path.
 */
hipError_t gfx906_fa_amd_rope_cache_write_kv(
    void *query, void *key, const void *value, int dtype, const int64_t *positions,
    const void *cos_sin_cache, int cos_sin_dtype, int64_t cos_sin_stride, int max_position,
    int rot_dim, int is_neox, const int64_t *slot_mapping, uint8_t *k_cache, uint8_t *v_cache,
    int num_tokens, int num_heads, int num_kv_heads, int head_size, int block_size,
    int64_t query_token_stride, int64_t query_head_stride, int64_t key_token_stride,
    int64_t key_head_stride, int64_t value_token_stride, int64_t value_head_stride,
    int64_t cache_block_stride, int64_t cache_head_stride, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (5) Varlen direct-paged attention over the planar Q8 K+V cache: decode,
 *     chunked prefill, mixed batches and speculative verify in one call.
 *
 *     q    [num_tokens, Hq, D] (element strides), dtype fp16/bf16/fp32.
 *     out  [num_tokens, Hq, D] (element strides), dtype fp32/fp16/bf16.
 *     Sequence s owns query tokens [query_start_loc[s], query_start_loc[s+1])
 *     and has seq_lens[s] cached tokens (the new ones included).
 *     Query row j of s sees keys k < seq_lens[s] with, when causal != 0,
 *       k <= q_abs_offset[s] + j   (q_abs_offset may be NULL: then
 *                                   q_abs_offset[s] = seq_lens[s] - n_q[s]).
 *     q-head hq reads kv-head hq / (Hq/Hkv).  A row with no visible key is 0.
 *     Numerics: dequantize-then-fp32 softmax (scores, max, sum and output
 *     accumulated in fp32; K int8 values enter the MFMA exactly and their
 *     scales are applied to the fp32 products; V scales are folded into P).
 *     Replaces gfx906_fa_launch_paged (extension/gfx906_fa_launcher.cu:222-352,
 *     declared at extension/gfx906_fa.cpp:63-90) and the host padding /
 *     unpadding of extension/gfx906_fa_paged.py:255-330.
 *     Requirements: D = 128, Hq % Hkv == 0, block_size % 16 == 0, cache
 *     strides and plane bases 16-byte aligned, max_query_len >= every n_q
 *     (it sizes the prefill grid; max_seq_len is advisory), and a workspace
 *     of at least gfx906_fa_amd_paged_attention_workspace_size(...) bytes,
 *     256-byte aligned (no initial contents needed: each call writes what it
 *     reads).  Calls sharing one workspace must be ordered (same stream).
 *     Decode-shaped sequences (n_q*Hq/Hkv <= 64 rows) are split stream-K
 *     style: the device's resident workgroups each stream an equal,
 *     contiguous share of all their 16-token KV sub-pages; segments cut
 *     between workgroups leave partial (m, l, O) in the workspace and a
 *     second kernel merges them.
 *     A prefill call also takes room for its 64-key tiles dequantized once
 *     to fp16 (35840 bytes per tile and kv-head, every prefill sequence at
 *     max_seq_len keys, at most 1 GiB): the tiles are then written once and
 *     copied into LDS by every workgroup that reads them.  Any workspace of
 *     at least plan_info()'s img_offset bytes runs the same call; when the
 *     images do not fit the room it has, the prefill workgroups dequantize
 *     each tile themselves (same outputs, bit for bit).
 */
size_t gfx906_fa_amd_paged_attention_workspace_size(int num_seqs, int num_tokens,
                                                    int num_heads, int num_kv_heads,
                                                    int head_size, int max_query_len,
                                                    int max_seq_len);

/* (5-bound) Workspace bytes that cover every call of (5) / (5b) on the
 *     current device with num_seqs <= max_num_seqs and num_tokens <=
 *     max_num_tokens, whatever max_query_len and the mix of decode,
 *     speculative-verify and prefill sequences: what a serving loop reserves
 *     once, before graph capture, for a layer's (num_heads, num_kv_heads)
 *     (the prefill tile-image room at its 1 GiB cap included).
 *     No reference counterpart (the reference grows its buffers per call,
 *     extension/gfx906_fa_backend.py:316-403). */
size_t gfx906_fa_amd_paged_attention_workspace_bound(int max_num_seqs, int64_t max_num_tokens,
                                                     int num_heads, int num_kv_heads,
                                                     int head_size);

/* (5-info) The launch plan of a call shape, for tests and diagnostics:
 *     info[0] workspace bytes, [1] decode classes, [2] largest decode row
 *     bound, [3] prefill kernel launched, [4] prefill row tiles (bound),
 *     [5] prefill work-list capacity, [6] split row tiles (bound), [7]
 *     partial slots per kv-head, [8] byte offset in the workspace of the
 *     prefill work-list header (int32 item count, int32 split row tile count,
 *     int32 1 if the tiles were dequantized once as images, int32 image
 *     tiles per kv-head; written by the call; -1 without a work list), [9]
 *     CUs planned for, [10] the workspace bytes every call needs (the image
 *     room starts there), [11] the image room (info[0] = [10] + [11]),
 *     [12] query rows per prefill row tile (256, or 128 for the
 *     key-interleaved tiles chosen when the longest prefill sequence has at
 *     most 128 rows per kv-head; 0 without a prefill launch).
 *     Returns the number of entries (13; at most info_len are written), or
 *     -1 for an invalid shape.  No reference counterpart. */
int gfx906_fa_amd_paged_attention_plan_info(int num_seqs, int num_tokens, int num_heads,
                                            int num_kv_heads, int head_size, int max_query_len,
                                            int max_seq_len, int64_t *info, int info_len);

/* (5-bound-info) The bound of (5-bound) in its two parts: info[0] the
 *     regions every call of those limits needs (each call's plan_info()
 *     img_offset is at most this), info[1] the room for prefill tile
 *     images of contexts up to max_seq_len keys (max_seq_len <= 0: any
 *     context, the library's 1 GiB cap).  The image room is optional: a
 *     workspace of info[0] bytes runs every such call, whose prefill
 *     workgroups then dequantize their own tiles where images do not fit.
 *     Returns 2 (at most info_len entries written) or -1 for an invalid
 *     shape.  No reference counterpart. */
int gfx906_fa_amd_paged_attention_workspace_bound_info(int max_num_seqs, int64_t max_num_tokens, int num_heads,
                                                       int num_kv_heads, int head_size, int64_t max_seq_len,
                                                       int64_t *info, int info_len);

/* Compute units of the current device the plans are made for (256, the
 * MI355X count, when no device is visible).  No reference counterpart. */
int gfx906_fa_amd_device_cus(void);

hipError_t gfx906_fa_amd_paged_attention(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
    int head_size, int block_size, int max_query_len, int max_seq_len, float scale,
    void *out, int out_dtype, int64_t out_token_stride, int64_t out_head_stride,
    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* (5n) (5) with no workspace argument and no allocation of any kind.  No
 *      counterpart in the reference: it is for callers that cannot allocate
 *      (code under HIP graph capture, tight serving loops, harnesses that
 *      forbid hipMalloc).  The workspace is the library's own scratch, a
 *      file-scope device array of GFX906_FA_AMD_SCRATCH_BYTES (64 MiB), one
 *      copy per device, held by every device the library runs on until the
 *      process ends.  Decode / verify plans are those of (5), so outputs
 *      are bit-identical to (5); a batch whose split-prefill partials would
 *      not fit in the scratch runs its prefill row tiles unsplit (same
 *      tolerance, different summation order); prefill tile images are
 *      written only when they fit the scratch past the plan (otherwise the
 *      prefill workgroups dequantize their own tiles, same bytes).  A batch
 *      whose plan still
 *      exceeds the scratch is rejected (hipErrorInvalidValue and a line on
 *      stderr) before any work is enqueued.  Every call on a device shares
 *      that device's scratch: calls that overlap on one device (concurrent
 *      streams, several host threads) race and must be ordered by the
 *      caller. */
#define GFX906_FA_AMD_SCRATCH_BYTES ((size_t)64 << 20)

hipError_t gfx906_fa_amd_paged_attention_noalloc(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
    int head_size, int block_size, int max_query_len, int max_seq_len, float scale,
    void *out, int out_dtype, int64_t out_token_stride, int64_t out_head_stride,
    hipStream_t stream);

/* (5n-copy) Diagnostics for (5n): copies `bytes` of the current device's
 *      scratch, from byte `offset`, to the device buffer `dst` (an ordinary
 *      stream-ordered copy).  With plan_info()'s work-list header offset it
 *      shows which prefill path the last (5n) call took.  Offsets past the
 *      scratch are refused (hipErrorInvalidValue).  No reference
 *      counterpart. */
hipError_t gfx906_fa_amd_noalloc_scratch_copy(void *dst, size_t offset, size_t bytes, hipStream_t stream);

/* (5b) (4) followed by (5) in one call: key / value [num_tokens, Hkv, D] (the
 *      query dtype, element strides) are quantized to Q8_0 and written at
 *      slot_mapping[t] (< 0 = skip) before attention reads the cache.  When
 *      every sequence is decode-shaped (n_q*Hq/Hkv <= 64 rows) and
 *      q_abs_offset is NULL, the new tokens are the last n_q positions of
 *      their sequences and the decode kernel itself quantizes each one in the
 *      wave that streams its sub-page, uses those bytes for attention and
 *      stores them - one launch fewer per decode step; otherwise (4) runs
 *      first.  The cache bytes and the output equal those of (4) then (5) on
 *      the same inputs, provided slot_mapping puts each new token at its
 *      position in block_table (as vLLM's metadata does).
 *      Replaces the reference's do_kv_cache_update + forward pair for decode
 *      steps (extension/gfx906_fa_backend.py:405-461), which the backend
 *      issues as two launches.
 */
hipError_t gfx906_fa_amd_paged_attention_kv_write(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
    int head_size, int block_size, int max_query_len, int max_seq_len, float scale,
    void *out, int out_dtype, int64_t out_token_stride, int64_t out_head_stride,
    void *workspace, size_t workspace_bytes, const void *key, const void *value,
    int kv_dtype, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t *slot_mapping,
    hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (6) Repack the reference's contiguous attention inputs for (7):
 *       k_aos [rows, Skv, 136] AoS Q8_0 K rows -> k_planar [rows, Skv_pad/16, 2176]
 *       v_f16 [rows, Skv, 128] fp16 V rows     -> v_planar [rows, Skv_pad/16, 4096]
 *     rows = B * Hkv (sequence-major), Skv_pad = Skv rounded up to 16; the
 *     padding tokens are written as zeros.  K bytes are permuted, never
 *     changed.  fp16 V sub-page layout: element (t, d) at byte
 *       2048*(d/64) + 32*(16*(t/4) + d%16) + 8*((d/16)%4) + 2*(t%4).
 *     Serves the contiguous entry gfx906_fa_forward
 *     (extension/gfx906_fa.cpp:120-265, launcher extension/gfx906_fa_launcher.cu:53-209),
 *     whose V stays fp16.
 */
hipError_t gfx906_fa_amd_pack_flat_kv(const uint8_t *k_aos, const void *v_f16,
                                      uint8_t *k_planar, void *v_planar, int rows, int Skv,
                                      int head_size, hipStream_t stream);

/* (7) Tiled paged attention with a choice of V plane and an optional
 *     additive mask; every sequence runs through the tiled (prefill) kernel,
 *     no workspace, fp32 output.
 *       v_format 0: planar Q8 V (as (5)); 1: planar fp16 V (layout of (6)).
 *       K / V page and kv-head strides in bytes, given separately.
 *       mask: NULL, or fp16 [num_seqs][n_q][mask_cols] with element strides
 *       mask_batch_stride / mask_row_stride: score(j, k) += mask[s][j][k]
 *       (natural-log units, added after the softmax scale as
 *       kernel/fattn-q8.cuh:643-644 does); keys k >= mask_cols add 0.
 *     Semantics otherwise as (5): dequantized K, exact fp16 (format 1) or
 *     dequantized Q8 (format 0) V, fp32 softmax, kv cutoff seq_lens[s],
 *     causal bound q_abs_offset (or seq_lens - n_q) when causal != 0.
 *     With (6), block_size = Skv_pad and one page per sequence this is the
 *     contiguous attention of gfx906_fa_launch
 *     (extension/gfx906_fa_launcher.cu:53-209); with v_format 0 it is the
 *     masked form of gfx906_fa_launch_paged
 *     (extension/gfx906_fa_launcher.cu:222-352).
 */
hipError_t gfx906_fa_amd_paged_attention_tiled(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const void *v_cache, int v_format, int64_t k_block_stride,
    int64_t k_head_stride, int64_t v_block_stride, int64_t v_head_stride,
    const int32_t *block_table, int64_t block_table_stride, const int32_t *seq_lens,
    const int32_t *query_start_loc, const int32_t *q_abs_offset, int causal,
    const void *mask, int64_t mask_batch_stride, int64_t mask_row_stride, int mask_cols,
    int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, float scale, float *out, int64_t out_token_stride,
    int64_t out_head_stride, hipStream_t stream);

/* (7) Contiguous decode: the decode shapes of gfx906_fa_launch
 *     (extension/gfx906_fa_launcher.cu:53-209; gfx906_fa.forward with
 *     seq_q * num_heads / num_kv_heads <= 16 and no mask) on the reference's
 *     own contiguous layouts, with no repacking pass: k_q8 AoS Q8_0 rows
 *     [batch][num_kv_heads][seq_kv][136 B], v_f16 fp16 rows
 *     [batch][num_kv_heads][seq_kv][128] (both 16-byte aligned, contiguous),
 *     q [batch * seq_q][num_heads][128] (element strides; dtype 0/1/2),
 *     kv_len int32 [batch] (keys each batch row sees, clamped to
 *     [0, seq_kv]), q_abs_offset int32 [batch] or NULL (row j sees keys
 *     k <= q_abs_offset[b] + j), out fp32 [batch * seq_q][num_heads][128]
 *     (element strides).  Each (batch, kv-head) is split over the keys into
 *     pieces (one single-wave workgroup each) merged by a second launch;
 *     workspace: gfx906_fa_amd_flat_decode_workspace_size() bytes (16-byte
 *     aligned; no initial contents).  Other shapes are refused
 *     (hipErrorInvalidValue and a line on stderr). */
size_t gfx906_fa_amd_flat_decode_workspace_size(int batch, int seq_q, int num_heads, int num_kv_heads,
                                                int seq_kv);
hipError_t gfx906_fa_amd_flat_decode(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride, const uint8_t *k_q8,
    const void *v_f16, const int32_t *kv_len, const int32_t *q_abs_offset, int batch, int seq_q, int num_heads,
    int num_kv_heads, int seq_kv, int head_size, float scale, float *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Measurement helper: streams `bytes` (a multiple of 16) from the 16-byte
 * aligned device buffer `src` with non-temporal 16-byte loads and writes one
 * XOR word per wave to `out` (at least gfx906_fa_amd_stream_read_words()
 * words).  Its rate is the read-only streaming ceiling the read-dominated
 * attention passes are compared with.  No reference counterpart. */
int gfx906_fa_amd_stream_read_words(void);
hipError_t gfx906_fa_amd_stream_read(const void *src, int64_t bytes, uint32_t *out, int out_words,
                                     hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* GFX906_FA_AMD_H */
