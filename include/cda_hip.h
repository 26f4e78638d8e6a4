/*
 * cda_hip.h -- C ABI of libcda_hip.so, the MI355X (gfx950) kernels of
 * Compressed-Domain Attention (CDA).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as `void *` (NULL = the default stream), launches asynchronously on
 * that stream, allocates nothing, and returns 0 on success or a negative
 * CDA_E_* code; cda_hip_last_error() then describes the failure (the message
 * is per thread).  Outputs are caller-allocated and written in place, as in
 * the reference's pybind functions.  All kernels are graph-capturable.
 *
 * Layouts shared by all entry points
 *   head_dim D = 128.
 *   Paged cache: flat (num_slots, H_kv, slot_bytes) uint8, slot index =
 *   block_table[b][t / block_size] * block_size + t % block_size.
 *   Slot = [K codes kb | V codes kb | K norm fp32 | V norm fp32 | pad],
 *   kb = D*bits/8: K4V4 (16 levels) kb=64, slot_bytes 144 (cda_attn_v2.py:20-60);
 *   K2V2 (4 levels) kb=32, slot_bytes 80.  Codes are packed MSB-first
 *   (compression.py:163-179, 375-386).  slot_bytes must be a multiple of 16.
 *   fp16 tensors are IEEE binary16 (passed as `void *`).
 */
#ifndef CDA_HIP_H
#define CDA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    CDA_OK = 0,
    CDA_E_INVALID = -1,   /* bad argument (shape, size, alignment, null) */
    CDA_E_HIP = -2,       /* HIP runtime error while launching */
    CDA_E_WORKSPACE = -3, /* workspace too small */
};

/* Library version (major*10000 + minor*100 + patch) and last error text. */
int cda_hip_version(void);
const char *cda_hip_last_error(void);

/* ---------------------------------------------------------------- decode --
 * Replaces the reference pybind function
 *   cda_decode_full_hmma_v3(Q, kv_cache, block_table, seq_lens, cb_K, cb_V,
 *                           rotation_fp32, rotation_fp16, out, group_size,
 *                           block_size, tile_N, max_seq_len, scale)
 * bound by cda/kernels_cuda/wrappers.py:115-124 (module
 * _v1_decode_hmma_k4v4_gs{4,8}, hmma_loader.py:27-32).
 *
 * q:            (B, H_q, 128) fp16, unrotated, contiguous.
 * kv_cache:     paged cache (see above), num_slots rows.
 * block_table:  (B, bt_stride) int32.       seq_lens: (B,) int32 (past + 1).
 * cb_k, cb_v:   (levels,) fp32 codebooks, levels = 16 (K4V4) or 4 (K2V2).
 * rot_f32:      (128, 128) fp32 rotation R; q_rot = fp16(q @ R) and
 *               out = fp16(fp16(O_rot) @ R^T) (compression.py:287-296).
 * rot_f16:      accepted for signature parity, not read.
 * out:          (B, H_q, 128) fp16, written in place.
 * group_size:   H_q / H_kv, 4 or 8.
 * tile_n:       context tokens per split-K partition; <= 0 selects the
 *               MI355X default (cda_decode_plan).  Rounded up to 32.
 * max_seq_len:  upper bound of seq_lens (sizes the split grid).
 * workspace:    device scratch of at least cda_decode_workspace_size(...)
 *               bytes, 256-byte aligned.
 */
int cda_decode_plan(int B, int H_q, int H_kv, int max_seq_len, int tile_n, int *tile_n_out,
                    int *n_splits_out);
size_t cda_decode_workspace_size(int B, int H_q, int H_kv, int max_seq_len, int tile_n);
/* Plan of the single-launch decode (no reference counterpart; the reference's
 * wrapper only sizes tile_N): workgroups of one KV head over 8 * wave_tokens
 * context tokens, n_splits per sequence.  wave_tokens is a multiple of 64,
 * 8 * wave_tokens <= 65536, and n_splits never exceeds cda_decode_plan's for
 * the same shape, so the single launch fits cda_decode_workspace_size(). */
int cda_decode_fused_plan(int B, int H_kv, int max_seq_len, int *wave_tokens_out,
                          int *n_splits_out);
int cda_decode_full_hmma_v3(const void *q, const void *kv_cache, int64_t num_slots,
                            int slot_bytes, int H_kv, const int32_t *block_table,
                            int bt_stride, const int32_t *seq_lens, const float *cb_k,
                            const float *cb_v, int levels, const float *rot_f32,
                            const void *rot_f16, void *out, int B, int H_q, int group_size,
                            int block_size, int tile_n, int max_seq_len, float scale,
                            void *workspace, size_t workspace_bytes, void *stream);

/* The legacy K4V2 cache (cda_attn_v2.py:29: "legacy K4V2 layout (104 B/slot)"):
 * slot = [K codes 4-bit 64 B | V codes 2-bit 32 B | K norm fp32 | V norm fp32],
 * 104 bytes (slot_bytes >= 104, a multiple of 8); cb_k has 16 levels, cb_v 4.
 * Replaces the module of load_decode_hmma(k4v2=True) (_v1_decode_hmma_k4v2_gs{4,8},
 * hmma_loader.py:27-32), same arguments as cda_decode_full_hmma_v3 with the
 * level count implied.  Runs the general split kernel. */
int cda_decode_full_hmma_v3_k4v2(const void *q, const void *kv_cache, int64_t num_slots,
                                 int slot_bytes, int H_kv, const int32_t *block_table,
                                 int bt_stride, const int32_t *seq_lens, const float *cb_k,
                                 const float *cb_v, const float *rot_f32, const void *rot_f16,
                                 void *out, int B, int H_q, int group_size, int block_size,
                                 int tile_n, int max_seq_len, float scale, void *workspace,
                                 size_t workspace_bytes, void *stream);

/* Decode with the score-domain QK of the reference's
 * qk_scores_uniform_4bit_without_k_decode / attention_compressed_rotated_
 * reference_qk_without_k_decode (cda/algorithm/attention.py:101-187) for a
 * K4V4 cache whose K codebook is the 16-level uniform one, cb[i] = (2i+1)/16 - 1
 * (compression.py:75-83): score = Kn * (q_rot . code / 8 - 15/16 sum(q_rot))
 * * scale from the integer codes (K never decoded), V decoded as fp16(cb_v *
 * Vn).  The reference has no kernel for it (its torch function is the
 * contract).  Same arguments as cda_decode_full_hmma_v3 (levels 16 implied,
 * no fp16 rotation); needs H_kv = 8, 144-byte slots and splits of at most
 * 16384 tokens (CDA_E_INVALID otherwise).  cb_k is checked on the device: if
 * it is not the uniform codebook the output is NaN. */
int cda_decode_full_hmma_v3_uniform_qk(const void *q, const void *kv_cache, int64_t num_slots,
                                       int slot_bytes, int H_kv, const int32_t *block_table,
                                       int bt_stride, const int32_t *seq_lens, const float *cb_k,
                                       const float *cb_v, const float *rot_f32, void *out, int B,
                                       int H_q, int group_size, int block_size, int tile_n,
                                       int max_seq_len, float scale, void *workspace,
                                       size_t workspace_bytes, void *stream);

/* Score-domain QK scores over contiguous compressed K
 * (qk_scores_uniform_4bit_without_k_decode, cda/algorithm/attention.py:101-152):
 *   q_rot:  (B, H_q, M_q, 128) fp16, rotated frame
 *   k_idx:  (B, H_kv, M_k, 64) uint8, 4-bit codes MSB-first, 16-byte aligned
 *   k_norm: (B, H_kv, M_k) fp32
 *   out:    (B, H_q, M_q, key_end - key_start) fp32 =
 *           k_norm * (q_rot . code / 8 - 15/16 sum(q_rot)) * scale, -inf where
 *           causal and key_start + k > m + q_offset. */
int cda_qk_scores_uniform4(const void *q_rot, const void *k_idx, const float *k_norm,
                           float *out, int B, int H_q, int H_kv, int M_q, int group_size,
                           int64_t M_k, int64_t key_start, int64_t key_end, int64_t q_offset,
                           float scale, int causal, void *stream);

/* Allocation-free variant of cda_decode_full_hmma_v3.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under graph capture that must not call hipMalloc, tight serving loops,
 * harnesses that forbid allocation).  Same arguments and result as
 * cda_decode_full_hmma_v3 without the workspace: the split-K partials go to
 * a fixed per-GPU device array of the library, of
 * cda_decode_noalloc_max_workspace() bytes (16 MiB; held until the process
 * ends).  Shapes whose cda_decode_workspace_size() exceeds it return
 * CDA_E_WORKSPACE.  It calls no allocator.  Calls on one GPU share the
 * array, so calls that overlap on one GPU are not allowed: serialise them on
 * one stream (graph replays included); overlapping calls from several
 * streams or threads race on the partials and give wrong output. */
size_t cda_decode_noalloc_max_workspace(void);
int cda_decode_full_hmma_v3_noalloc(const void *q, const void *kv_cache, int64_t num_slots,
                                    int slot_bytes, int H_kv, const int32_t *block_table,
                                    int bt_stride, const int32_t *seq_lens, const float *cb_k,
                                    const float *cb_v, int levels, const float *rot_f32,
                                    const void *rot_f16, void *out, int B, int H_q,
                                    int group_size, int block_size, int tile_n,
                                    int max_seq_len, float scale, void *stream);

/* Profiling hook, no counterpart in the reference: when both are non-NULL,
 * later cda_decode_full_hmma_v3 calls on this thread record the two hipEvent_t
 * on the launch stream immediately before and after the split-K kernel (the
 * kernel that streams the cache), so a caller can time it alone.  Pass NULL,
 * NULL to stop. */
int cda_decode_set_timing_events(void *start_event, void *stop_event);

/* Selects the decode split kernel for later calls (process-wide; default 1).
 * enable=1 lets cda_decode_full_hmma_v3 use the page-streaming kernel when the
 * cache is 8 KV heads x 144-byte (K4V4) or 80-byte (K2V2) slots and the K and
 * V codebooks hold equal bits (one pointer, or two compared on the device);
 * enable=0 always takes the general kernel.  Both produce the same result to
 * fp32 rounding of the softmax sums.  No reference counterpart: the reference
 * has one decode kernel; this exists for A/B measurement and tests. */
int cda_decode_set_stream_kernel(int enable);

/* Selects the single-launch decode for later calls (process-wide; default 1).
 * enable=1 lets cda_decode_full_hmma_v3 run, where the page-streaming kernel
 * applies with one codebook pointer for K and V and the library's split plan
 * (tile_n = 0, or the tile_n that cda_decode_plan returns for tile_n = 0, which
 * is what the reference-shaped wrapper passes), one kernel per call: each workgroup takes one KV head over a token
 * range, rotates q itself, merges its waves' partials and, when its range is
 * the whole sequence, writes out (otherwise combine_kernel follows).  The
 * timing events above then bracket that kernel.  enable=0 keeps the
 * rotate / split / combine launches.  No reference counterpart: for A/B
 * measurement and tests. */
int cda_decode_set_fused_kernel(int enable);

/* ---------------------------------------------------------------- encode --
 * Replaces the reference pybind function
 *   cda_paged_encode_fused(K, V, slot_mapping, flat_cache, cb_K, cb_V)
 * bound by cda/kernels_cuda/wrappers.py:153-156 (module
 * _v1_paged_encode_fused, hmma_loader.py:35-37).
 *
 * k, v:          (T, H_kv, 128) fp16 unrotated, row stride k_stride/v_stride
 *                elements between tokens (heads contiguous).
 * slot_mapping:  (T,) int32; a negative slot (vLLM padding) is skipped.
 * flat_cache:    (num_slots, H_kv, slot_bytes) uint8, written in place.
 * cb_k, cb_v:    (levels,) fp32, levels = 16 (K4V4) or 4 (K2V2).
 * Per (token, head, role), bit-identical to Compressor.encode
 * (compression.py:315-335) on the CPU: Hadamard-128 as the fp32 fma chain
 * over k in order rounded to fp16, fp32 L2 norm in eight ordered lane sums
 * clamped to 1e-12, nearest centroid with ties to the lower index (codebooks
 * sorted ascending, as bucketize requires), MSB-first packing.
 */
int cda_paged_encode_fused(const void *k, const void *v, int64_t k_stride, int64_t v_stride,
                           const int32_t *slot_mapping, int64_t num_tokens, void *flat_cache,
                           int64_t num_slots, int slot_bytes, int H_kv, const float *cb_k,
                           const float *cb_v, int levels, void *stream);

/* cda_paged_encode_fused into the legacy K4V2 slot (104 B, layout above the
 * K4V2 decode): K with the 16-level cb_k, V with the 4-level cb_v.  Replaces
 * the K4V2 cache-update module (_v1_kv_update_k4v2, hmma_loader.py:40-43;
 * the reference names it but no caller shows its symbol, so it takes the
 * fused encode's arguments). */
int cda_paged_encode_fused_k4v2(const void *k, const void *v, int64_t k_stride,
                                int64_t v_stride, const int32_t *slot_mapping,
                                int64_t num_tokens, void *flat_cache, int64_t num_slots,
                                int slot_bytes, int H_kv, const float *cb_k, const float *cb_v,
                                void *stream);

/* --------------------------------------------------------------- prefill --
 * Causal varlen prefill with the Hadamard-128 rotation of Q fused in front and
 * the inverse rotation of O fused behind (bottom-right causal alignment:
 * key k is visible to query i of sequence b iff k <= i + seq_k[b] - seq_q[b]).
 * O_rot is rounded to fp16 before the inverse rotation (attention.py:93).
 *
 * cda_prefill_paged_hadamard reads K/V straight from the compressed K4V4
 * paged cache (tiles are dequantised into LDS, no dense scratch).  It replaces
 * the pair paged_cache_to_dense_rotated + cda_fa2_varlen_fwd_hadamard that
 * fa2_cda_prefill_varlen_v1(fuse_fa2_epilogue=True) runs
 * (cda/kernels_cuda/fa2_cda.py:98-230).  No single reference symbol.
 *   q, out:        (T, H_q, 128) fp16, unrotated; T = cu_seqlens_q[B] (a larger
 *                  T leaves the extra out rows untouched; query rows past T
 *                  are neither read nor written).
 *   cu_seqlens_q:  (B+1,) int32.   seq_lens: (B,) int32 key lengths.
 *   H_q / H_kv:    4 or 8.         levels: 16.
 *   block_size:    a multiple of 16 (pages of 16 tokens or more).
 */
int cda_prefill_paged_hadamard(const void *q, const void *kv_cache, int64_t num_slots,
                               int slot_bytes, int H_kv, const int32_t *block_table,
                               int bt_stride, const int32_t *cu_seqlens_q,
                               const int32_t *seq_lens, int B, const float *cb_k,
                               const float *cb_v, int levels, void *out, int T, int H_q,
                               int block_size, int max_query_len, float scale, void *stream);

/* Same operation as cda_prefill_paged_hadamard, for short query chunks over
 * long contexts: when the query blocks x sequences x KV heads leave most CUs
 * idle (fewer than 256 workgroups), the keys of each query block are split
 * (at least 256 keys per split, at most 64 splits); the splits write
 * unnormalised partials (O, m, l) into the workspace and a combine kernel
 * merges them (attention.py:239-272) before the fp16 rounding of O_rot and
 * the inverse rotation.  When no split pays it runs the unsplit kernel and
 * ignores the workspace.  Same reference call site as above
 * (fa2_cda.py:98-230; the reference has no split form).
 *   max_seq_len:   upper bound of seq_lens[b] (the longest key range).
 *   workspace:     device scratch, 256-byte aligned, of at least
 *                  cda_prefill_workspace_size(B, T, H_q, H_kv, max_query_len,
 *                  max_seq_len) bytes (0: no split, workspace may be NULL).
 * Calls sharing one workspace must not overlap.
 */
size_t cda_prefill_workspace_size(int B, int T, int H_q, int H_kv, int max_query_len,
                                  int max_seq_len);
int cda_prefill_paged_hadamard_ws(const void *q, const void *kv_cache, int64_t num_slots,
                                  int slot_bytes, int H_kv, const int32_t *block_table,
                                  int bt_stride, const int32_t *cu_seqlens_q,
                                  const int32_t *seq_lens, int B, const float *cb_k,
                                  const float *cb_v, int levels, void *out, int T, int H_q,
                                  int block_size, int max_query_len, int max_seq_len, float scale,
                                  void *workspace, size_t workspace_bytes, void *stream);

/* Replaces the reference's hybrid chunked prefill
 *   hybrid_attn_v1(q, k, v, output, kv_cache_flat, block_table, cu_seqlens_q=,
 *                  seq_lens=, cb_K=, cb_V=, rotation_fp32=, rotation_fp16=,
 *                  scale=, group_size=, block_size=)
 * called by cda/kernels_cuda/vllm_integration/cda_attn_v2.py:1023-1060 and
 * :1474-1532 (CDA_PREFILL_BACKEND fa2_rawkv / fa2_cda_rawkv /
 * fa2_cda_fused_rawkv with a compressed prefix; the reference's own wrapper was
 * removed, wrappers.py:14-20).  Sequence b's queries are the last
 * q_len = cu_seqlens_q[b+1] - cu_seqlens_q[b] of its seq_lens[b] positions.
 * They attend to keys [0, seq_lens[b] - q_len) of the compressed cache (all
 * visible) and to the chunk's own fresh keys k_new / v_new rows
 * [cu_seqlens_q[b], cu_seqlens_q[b+1]) (causal), in one softmax: the chunk's K
 * and V are rotated to fp16(x H / sqrt(128)) (fa2_cda.py:256-287), each source
 * writes split partials (O, m, l), and the merge (attention.py:239-272) rounds
 * O_rot to fp16 and applies the inverse rotation (when neither side needs a
 * key split, the prefix kernel merges the chunk's partial in its epilogue).
 *   q, out:         (T, H_q, 128) fp16, unrotated
 *   k_new, v_new:   (T, H_kv, 128) fp16, unrotated, contiguous
 *   kv_cache:       K4V4 paged cache (levels 16)
 *   max_seq_len:    upper bound of seq_lens (plans the splits only)
 *   workspace:      256-byte aligned device scratch of at least
 *                   cda_prefill_hybrid_workspace_size(...) bytes
 * Calls sharing one workspace must not overlap.
 */
size_t cda_prefill_hybrid_workspace_size(int B, int T, int H_q, int H_kv, int max_query_len,
                                         int max_seq_len);
int cda_prefill_hybrid_rawkv(const void *q, const void *k_new, const void *v_new,
                             const void *kv_cache, int64_t num_slots, int slot_bytes, int H_kv,
                             const int32_t *block_table, int bt_stride,
                             const int32_t *cu_seqlens_q, const int32_t *seq_lens, int B,
                             const float *cb_k, const float *cb_v, int levels, void *out, int T,
                             int H_q, int block_size, int max_query_len, int max_seq_len,
                             float scale, void *workspace, size_t workspace_bytes, void *stream);

/* Replaces the reference pybind function
 *   cda_fa2_varlen_fwd_hadamard(Q, k_rot, v_rot, out, cu_q, cu_k, seqused_k,
 *                               max_q, max_k, scale)      (causal only)
 * bound by cda/kernels_cuda/fa2_cda.py:166-181 (module _v1_fa2_cda_varlen_fused,
 * hmma_loader.py:56-58).  k_rot, v_rot: dense rotated fp16 rows
 * (rows, H_kv, 128); sequence b's keys are rows cu_seqlens_k[b] ..
 * cu_seqlens_k[b] + seqused_k[b] - 1. */
int cda_fa2_varlen_fwd_hadamard(const void *q, const void *k_rot, const void *v_rot, void *out,
                                const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                                const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                                int max_query_len, int max_seq_len, float scale, void *stream);

/* Comparator kernels behind the FA2-fork torch.ops namespace
 * (torch.ops._cda_vllm_fa2_fork_C, cda/kernels_vllm_fa2_fork/interface.py:
 * 138-162, 234-257, 304-328, 434-461); they carry no Hadamard rotation, all
 * tensors are in one frame.
 *
 * cda_fa2_varlen_fwd: the flash attention of cda_fa2_varlen_fwd_hadamard
 * without the prologue/epilogue rotation, causal (bottom-right) or not
 * (causal = 0: every key of the sequence visible).  Dense fp16 K/V rows. */
int cda_fa2_varlen_fwd(const void *q, const void *k, const void *v, void *out,
                       const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                       const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                       int max_query_len, float scale, int causal, void *stream);

/* cda_fa2_varlen_fwd_lse: cda_fa2_varlen_fwd that also writes the softmax
 * log-sum-exp the fork's varlen ops return beside out
 * (cda/kernels_vllm_fa2_fork/interface.py:234-258, 304-329, 434-470):
 * softmax_lse (H_q, T) fp32, softmax_lse[h][t] = log(sum over query t's
 * visible keys of exp(scale * q.k)), +inf for a query with no visible key
 * (FlashAttention-2's varlen layout and convention). */
int cda_fa2_varlen_fwd_lse(const void *q, const void *k, const void *v, void *out,
                           const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                           const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                           int max_query_len, float scale, int causal, float *softmax_lse,
                           void *stream);

/* cda_dequantize_rows: out row r = fp16(cb[code] * norm) (compression.py:
 * 337-361, rotated frame) of code rows (rows, H, 64 or 32 bytes) and norms
 * (rows, H) fp32 -- the reference fork's dequantize_compressed_kv for one of
 * K or V.  With block_table != NULL the codes/norms are a paged pool and
 * out is (B * max_seq_len, H, 128): row b*max_seq_len + t = token t of
 * sequence b (slot block_table[b][t / block_size] * block_size +
 * t % block_size), zeros past seq_lens[b]; rows must equal B * max_seq_len. */
int cda_dequantize_rows(const void *codes, const float *norms, int64_t rows, int H,
                        const float *cb, int levels, const int32_t *block_table, int bt_stride,
                        const int32_t *seq_lens, int block_size, int max_seq_len, void *out,
                        void *stream);

/* Replaces the reference pybind function
 *   cda_fa2_paged_cache_to_dense_rotated(kv, block_table, seq_lens, cb_K, cb_V,
 *                                        block_size, max_seq_len) -> (k_rot, v_rot)
 * bound by cda/kernels_cuda/fa2_cda.py:85-95 (module _v1_fa2_cda_loader_k4v4,
 * hmma_loader.py:45-48).  Writes k_out, v_out: (B * max_seq_len, H_kv, 128)
 * fp16, row b*max_seq_len + t = fp16(centroid * norm) for t < seq_lens[b],
 * zeros beyond.  K4V4 only. */
int cda_fa2_paged_cache_to_dense_rotated(const void *kv_cache, int64_t num_slots, int slot_bytes,
                                         int H_kv, const int32_t *block_table, int bt_stride,
                                         const int32_t *seq_lens, int B, const float *cb_k,
                                         const float *cb_v, int levels, int block_size,
                                         int max_seq_len, void *k_out, void *v_out,
                                         void *stream);

/* cda_fa2_paged_cache_to_dense_rotated for the legacy K4V2 cache (the module
 * of load_fa2_cda_loader(k4v2=True), _v1_fa2_cda_loader_k4v2,
 * hmma_loader.py:46-49, called by fa2_cda.py:64-95): V rows decoded from the
 * 2-bit codes with the 4-level cb_v. */
int cda_fa2_paged_cache_to_dense_rotated_k4v2(const void *kv_cache, int64_t num_slots,
                                              int slot_bytes, int H_kv,
                                              const int32_t *block_table, int bt_stride,
                                              const int32_t *seq_lens, int B, const float *cb_k,
                                              const float *cb_v, int block_size,
                                              int max_seq_len, void *k_out, void *v_out,
                                              void *stream);

/* Replaces the reference pybind function hadamard128_fp16(x, y, scale)
 * (cda/kernels_cuda/fa2_cda.py:51-52, module _v1_fa2_cda_hadamard128):
 * y = fp16(scale * x @ H_128) for `rows` rows of 128 fp16, H the unnormalised
 * Sylvester matrix (natural order). */
int cda_hadamard128_fp16(const void *x, void *y, int64_t rows, float scale, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* CDA_HIP_H */
