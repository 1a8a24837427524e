/*
 * kvpath.h - C ABI of the MI355X (gfx950) paged KV-cache library, libkvpath.so.
 *
 * The library implements the three device operations of Kavor's paged KV-cache
 * path:
 *
 *   kvp_append_bf16          replaces the Triton kernel store_kvcache_kernel and its
 *                            wrapper store_kvcache
 *                            (kavor/layers/attention/flash_attention_kvcache.py:10-46)
 *   kvp_paged_decode_bf16    replaces flash_attn_with_kvcache(q.unsqueeze(1), k_cache,
 *                            v_cache, cache_seqlens, block_table, softmax_scale,
 *                            causal=True)  (flash_attention_kvcache.py:80-83)
 *   kvp_varlen_prefill_bf16  replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q,
 *                            cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
 *                            causal=True, block_table)  (flash_attention_kvcache.py:73-79)
 *
 * Conventions shared by every entry point:
 *   - Tensors are passed as a device pointer plus element strides (not bytes).
 *     bf16 data is passed as void*; the innermost (head_dim) stride is always 1.
 *   - A paged cache is [num_blocks, block_size, num_kv_heads, head_dim] with strides
 *     (block_stride, slot_stride, head_stride, 1).  K and V share one stride set; in
 *     Kavor's page pool K and V are interleaved per page, so block_stride is
 *     2*block_size*num_kv_heads*head_dim (kavor/engine/cache_pool.py:311-322).
 *   - Every pointer must be 16-byte aligned and every stride a multiple of 8 elements
 *     (the kernels move 16-byte vectors).  head_dim must be 64, 128 or 256 for the
 *     append and 128 for attention.
 *   - Work is enqueued on `stream` (a hipStream_t; pass the current torch stream).
 *     Nothing is allocated, freed or synchronised, so every entry point may be
 *     captured into a hipGraph; all per-step metadata is read from device memory.
 *   - Return value: 0 on success, a negative KVP_E* code when the arguments are
 *     rejected on the host (nothing was launched), or a positive hipError_t when a
 *     launch failed.  kvp_last_error() describes the last failure on this thread.
 */
#ifndef KAVOR_AMD_KVPATH_H
#define KAVOR_AMD_KVPATH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVP_OK 0
#define KVP_EINVAL (-1)        /* bad shape, stride, alignment or null pointer */
#define KVP_EUNSUPPORTED (-2)  /* valid but not implemented (head_dim, GQA ratio) */
#define KVP_EWORKSPACE (-3)    /* decode workspace smaller than required */

/* Message for the last failing call on the calling thread ("" if none). */
const char* kvp_last_error(void);

/* Library version string, e.g. "kvpath 0.1 gfx950". */
const char* kvp_version(void);

/*
 * KV append: for token i with s = slot_mapping[i], copy key[i] (num_kv_heads x
 * head_dim) to k_cache[s / block_size, s % block_size] and value[i] to
 * v_cache[...] bit for bit.  s == -1 marks a padding token and is skipped; so is
 * any other s outside [0, num_cache_slots) (the reference leaves that undefined).
 * Replaces store_kvcache (flash_attention_kvcache.py:37-46), which takes the key
 * and value row strides separately (Qwen3: 1024 and 4096 elements,
 * kavor/models/qwen3.py:80-87) and one block stride for both caches.
 * Duplicate slots are allowed (graph capture writes slot 0 for every row); which
 * writer wins is unspecified, as in the reference.
 */
int kvp_append_bf16(const void* key, int64_t key_tok_stride, int64_t key_head_stride,
                    const void* value, int64_t value_tok_stride, int64_t value_head_stride,
                    void* k_cache, void* v_cache,
                    int64_t cache_block_stride, int64_t cache_slot_stride,
                    int64_t cache_head_stride, int64_t num_cache_slots,
                    const int32_t* slot_mapping, int32_t num_tokens,
                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                    void* stream);

/*
 * Bytes of device workspace kvp_paged_decode_bf16 needs for up to max_num_seqs
 * sequences whose block tables are max_blocks_per_seq wide with block_size-token
 * blocks.  The caller allocates it once (before any graph capture), 256-byte aligned,
 * and passes it on every call; its contents need no initialisation.  It holds the
 * batch's step prefix sums and the fp32 partial states of sequences that the
 * work split divides: at most (ranges + sequences) states per query head, with at most
 * 1024 ranges per launch, whatever the context lengths (Qwen3-0.6B, 512 sequences:
 * 12.8 MB).  Returns 0 for arguments the decode does not support.
 */
size_t kvp_decode_workspace_bytes(int32_t max_num_seqs, int32_t num_q_heads, int32_t head_dim,
                                  int32_t max_blocks_per_seq, int32_t block_size);

/*
 * Paged decode attention, one query token per sequence:
 *   out[b, h] = softmax(scale * q[b, h] . K_b^T) V_b
 * where K_b / V_b are the first context_lens[b] logical tokens of sequence b,
 * token t living at slot t % block_size of block block_tables[b, t / block_size],
 * and query head h reads kv head h / (num_q_heads / num_kv_heads) (GQA).
 * Replaces flash_attn_with_kvcache(..., causal=True) with one query token
 * (flash_attention_kvcache.py:80-83; the causal flag is a no-op for q_len 1).
 * Block-table entries at index >= ceil(context_lens[b] / block_size) are never
 * read (they are stale inside captured graphs, model_runner.py:235).
 * context_lens[b] == 0 writes zeros (graph padding rows).  A needed block id
 * outside [0, num_cache_blocks) or a context longer than
 * max_blocks_per_seq * block_size makes that sequence's output NaN instead of
 * reading out of bounds.  block_size must be a multiple of 64.
 * The output row of head h is out + b*out_seq_stride + h*out_head_stride (out
 * 16-byte aligned, both strides multiples of 8 elements).
 */
int kvp_paged_decode_bf16(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                          const void* k_cache, const void* v_cache,
                          int64_t cache_block_stride, int64_t cache_slot_stride,
                          int64_t cache_head_stride, int32_t num_cache_blocks,
                          const int32_t* block_tables, int64_t block_table_stride,
                          const int32_t* context_lens, int32_t num_seqs,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t max_blocks_per_seq,
                          float softmax_scale,
                          void* out, int64_t out_seq_stride, int64_t out_head_stride,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Decode step of a Qwen3 attention layer in one launch: q/k RMSNorm + neox RoPE of the
 * decode token, its K/V append, and paged decode attention.  Row b of qkv holds the token's
 * num_q_heads q heads, then num_kv_heads k heads, then num_kv_heads v heads (the fused
 * qkv projection output, kavor/models/qwen3.py:80-88).  For each sequence b the kernel
 *   - normalises and rotates its q heads and k heads with q_norm_weight / k_norm_weight
 *     and cos_sin at position context_lens[b] - 1, the decode token's position
 *     (kvp_qk_norm_rope_append_bf16's arithmetic; a position outside the table gives a
 *     NaN row);
 *   - appends the rotated k and the raw v at slot_mapping[b] (skipped for -1 or a slot
 *     outside the pool);
 *   - attends over context_lens[b] tokens (kvp_paged_decode_bf16's arithmetic), of which
 *     the last is this token: its k and v come from the qkv row, not from the cache, so
 *     the launch never reads a slot it writes.
 * slot_mapping[b] must be the slot of position context_lens[b] - 1 (as the engine builds
 * decode metadata, model_runner.py:448-460) for the result to equal the separate calls.
 * Rows without work (context 0, or longer than the block table) are not appended.  Replaces q_norm, k_norm, rotary_emb and Attention.forward's
 * store_kvcache + flash_attn_with_kvcache in decode (qwen3.py:85-90;
 * flash_attention_kvcache.py:71-83).  The workspace is kvp_paged_decode_bf16's.
 */
int kvp_paged_decode_fused_bf16(const void* qkv, int64_t qkv_tok_stride,
                                const float* cos_sin, int32_t max_position,
                                const void* q_norm_weight, const void* k_norm_weight, float eps,
                                void* k_cache, void* v_cache,
                                int64_t cache_block_stride, int64_t cache_slot_stride,
                                int64_t cache_head_stride, int32_t num_cache_blocks,
                                const int32_t* slot_mapping,
                                const int32_t* block_tables, int64_t block_table_stride,
                                const int32_t* context_lens, int32_t num_seqs,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int32_t max_blocks_per_seq, float softmax_scale,
                                void* out, int64_t out_seq_stride, int64_t out_head_stride,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * kvp_paged_decode_bf16 without a workspace argument: the decode's partial states live
 * in a static 32 MiB device array of the library (one per GPU, held until the process
 * ends), so the call allocates nothing and needs no caller buffer.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, semantics and results as kvp_paged_decode_bf16 (bit for bit).  A batch
 * whose partial states do not fit (about (R + num_seqs) * num_q_heads * 520 bytes, where
 * R <= 1024 is the launch's range count: the resident workgroups divided by
 * ceil(num_kv_heads / 4), so 512 with 8 kv heads and up to 1024 with 4 or fewer on
 * MI355X; Qwen3-0.6B at 512 sequences takes 8.5 MB) returns KVP_EWORKSPACE before any
 * launch.  Every call on one GPU shares that GPU's array, so calls that overlap on one
 * GPU (different streams or threads without ordering) race; calls ordered on one
 * stream do not.  The array needs no clearing between calls.  The array's device
 * address is looked up on the first call on each device, which must not be inside a
 * graph capture: such a first call returns KVP_EINVAL before any launch.  After one
 * call outside capture the entry point may be captured and replayed with new metadata
 * in the same buffers.
 */
int kvp_paged_decode_bf16_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                  const void* k_cache, const void* v_cache,
                                  int64_t cache_block_stride, int64_t cache_slot_stride,
                                  int64_t cache_head_stride, int32_t num_cache_blocks,
                                  const int32_t* block_tables, int64_t block_table_stride,
                                  const int32_t* context_lens, int32_t num_seqs,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int32_t max_blocks_per_seq,
                                  float softmax_scale,
                                  void* out, int64_t out_seq_stride, int64_t out_head_stride,
                                  void* stream);

/*
 * Variable-length prefill attention over packed sequences (bf16 MFMA).
 * Sequence s owns query rows [cu_seqlens_q[s], cu_seqlens_q[s+1]) of q and keys
 * 0 .. klen_s-1 with klen_s = cu_seqlens_k[s+1] - cu_seqlens_k[s].  With causal != 0
 * the mask is bottom-right aligned: query i (0-based within the sequence, qlen_s
 * queries) sees key j iff j <= i + klen_s - qlen_s (flash-attn >= 2.1 semantics;
 * the reference pins flash-attn 2.8.3.post2, setup.py:10).  Rows that see no key
 * are written as zeros.
 *
 * K/V source:
 *   block_tables == NULL  dense mode: key j of sequence s is row cu_seqlens_k[s] + j
 *                         of k / v ([total_k, num_kv_heads, head_dim]); the block
 *                         strides are ignored.
 *   block_tables != NULL  paged mode: k / v are the caches and key j of sequence s
 *                         lives at slot j % block_size of block
 *                         block_tables[s, j / block_size] (prefix-cached prefill,
 *                         flash_attention_kvcache.py:74-75).  A needed block id
 *                         outside [0, num_cache_blocks) or klen_s larger than
 *                         max_blocks_per_seq * block_size makes that sequence's
 *                         output NaN.  block_size must be a multiple of 64.
 *                         Every sequence has a row (block_table_stride apart) of
 *                         max_blocks_per_seq >= 1 entries; the first entry of each
 *                         row is read even for a sequence without queries (sequences
 *                         that start with the same block are scheduled together).
 * q, k, v and out are 16-byte aligned, head_dim is contiguous and every other stride is a
 * multiple of 8 elements (KVP_EINVAL otherwise).
 * max_seqlen_q only sizes the work list: a sequence longer than it is still computed in
 * full (its extra query tiles are taken by the workgroups that own its first ones), so
 * an understated max_seqlen_q costs time, never rows.  The workspace (size from
 * kvp_prefill_workspace_bytes, 256-byte aligned) holds the launch's work list; a smaller
 * one returns KVP_EWORKSPACE before any launch, and calls that share one workspace must
 * be ordered on one stream.  Replaces
 * flash_attn_varlen_func(..., causal=True, block_table) (flash_attention_kvcache.py:76-79).
 */
int kvp_varlen_prefill_bf16(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                            const void* k, int64_t k_block_stride, int64_t k_tok_stride,
                            int64_t k_head_stride,
                            const void* v, int64_t v_block_stride, int64_t v_tok_stride,
                            int64_t v_head_stride,
                            const int32_t* block_tables, int64_t block_table_stride,
                            int32_t num_cache_blocks, int32_t block_size,
                            int32_t max_blocks_per_seq,
                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                            int32_t num_seqs, int32_t max_seqlen_q,
                            int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                            float softmax_scale, int32_t causal,
                            void* out, int64_t out_tok_stride, int64_t out_head_stride,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace kvp_varlen_prefill_bf16 needs for up to num_seqs sequences
 * whose longest has max_seqlen_q query tokens (num_q_heads / num_kv_heads picks the
 * tile shape): 2 KiB plus 32 bytes per pair of query tiles per sequence, for at most
 * 2048 sequences (one launch; larger batches run as consecutive launches on the same
 * workspace).  Qwen3-0.6B, 256 sequences of up to 4096 tokens: 264 KiB.  The caller
 * allocates it once (before any graph capture), 256-byte aligned; it needs no
 * initialisation: every call rewrites what it reads.  Returns 0 for arguments the
 * prefill does not support.
 */
size_t kvp_prefill_workspace_bytes(int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                                   int32_t num_kv_heads);

/* ------------------------------------------------------------------------------
 * The layer work on either side of the path (the engine's Qwen3 layers).  Same
 * conventions as above.
 * ------------------------------------------------------------------------------ */

/*
 * RMSNorm over rows of a bf16 view: row (t, h), t < num_tokens, h < rows_per_token,
 * starts at x + t*x_stride0 + h*x_stride1 and has `cols` elements (a multiple of 8,
 * at most 8192).  With residual == NULL:
 *   out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)
 * (replaces RMSNorm.rms_forward / _rmsnorm_kernel, kavor/layers/layernorm.py:8-40,
 * 235-258).  With a residual (same indexing) the row is first summed in fp32,
 *   s = x + residual;  residual <- bf16(s);  out = bf16(bf16(s * rsqrt(mean(s^2)+eps)) * weight)
 * (replaces add_rms_forward / _add_rmsnorm_kernel, layernorm.py:113-140, 260-284; the
 * residual is updated in place as there).  out may alias x.
 */
int kvp_rmsnorm_bf16(const void* x, int64_t x_stride0, int64_t x_stride1,
                     void* residual, int64_t residual_stride0, int64_t residual_stride1,
                     const void* weight, float eps,
                     void* out, int64_t out_stride0, int64_t out_stride1,
                     int32_t num_tokens, int32_t rows_per_token, int32_t cols, void* stream);

/*
 * Fused per-token q/k RMSNorm + neox RoPE + KV append for head_dim 128.  Row t of qkv
 * holds num_q_heads q heads, then num_kv_heads k heads, then num_kv_heads v heads, each
 * head_dim contiguous elements (the fused qkv projection output, kavor/models/qwen3.py:80-88).
 * For each token:
 *   q_h = rope(rmsnorm(q_h, q_norm_weight))  written to q_out + t*q_out_tok_stride + h*128
 *   k_h = rope(rmsnorm(k_h, k_norm_weight))  written to the K cache at slot_mapping[t]
 *   v_h                                       copied bit for bit to the V cache there
 * rmsnorm is kvp_rmsnorm_bf16's formula; rope rotates pairs (x_i, x_{i+64}) of the bf16
 * normalised head by cos_sin[positions[t]] (a [max_position, 128] fp32 table holding
 * cos(p * theta_i) in columns 0..63 and sin in 64..127), in fp32, rounded once
 * (rotary_embedding.py:8-53, 104-120).  Cache addressing and slot semantics are
 * kvp_append_bf16's (slot -1 or outside [0, num_cache_slots) skips the token's k and v).
 * slot_mapping may be NULL (no append; the caches are then not touched).  A position
 * outside [0, max_position) makes that token's q and k NaN.  Replaces qwen3.py:85-89
 * (q_norm, k_norm, rotary_emb, then Attention's store_kvcache).
 */
int kvp_qk_norm_rope_append_bf16(const void* qkv, int64_t qkv_tok_stride,
                                 const int32_t* positions, const float* cos_sin,
                                 int32_t max_position,
                                 const void* q_norm_weight, const void* k_norm_weight, float eps,
                                 void* q_out, int64_t q_out_tok_stride,
                                 void* k_cache, void* v_cache,
                                 int64_t cache_block_stride, int64_t cache_slot_stride,
                                 int64_t cache_head_stride, int64_t num_cache_slots,
                                 const int32_t* slot_mapping, int32_t num_tokens,
                                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t block_size, void* stream);

/*
 * The same per-token q/k RMSNorm + neox RoPE without the append: q goes to q_out as
 * above and k to k_out + t*k_out_tok_stride + h*128 (a fresh [tokens, num_kv_heads, 128]
 * tensor); the v heads of qkv are not read.  Replaces q_norm, k_norm and rotary_emb
 * (kavor/models/qwen3.py:85-88; layernorm.py:8-40; rotary_embedding.py:8-53) for a
 * caller that then passes q, k and the v view of qkv to Attention.forward, which appends
 * k and v itself (flash_attention_kvcache.py:71-72).  qkv's row stride must cover the
 * q and k heads.
 */
int kvp_qk_norm_rope_bf16(const void* qkv, int64_t qkv_tok_stride,
                          const int32_t* positions, const float* cos_sin, int32_t max_position,
                          const void* q_norm_weight, const void* k_norm_weight, float eps,
                          void* q_out, int64_t q_out_tok_stride,
                          void* k_out, int64_t k_out_tok_stride,
                          int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, void* stream);

/*
 * out[t, i] = bf16(silu(gate[t, i]) * up[t, i]) with gate = gate_up[t, 0:intermediate],
 * up = gate_up[t, intermediate:2*intermediate], computed in fp32 and rounded once
 * (SiluAndMul, kavor/layers/activation.py:6-11, under torch.compile).  intermediate is a
 * multiple of 8.
 */
int kvp_silu_mul_bf16(const void* gate_up, int64_t gate_up_tok_stride, void* out,
                      int64_t out_tok_stride, int32_t num_tokens, int32_t intermediate,
                      void* stream);

/*
 * Greedy sampling: out[r] = index of the largest of logits[r, 0:vocab] (int64), the first
 * one on ties, NaN counting as largest (torch.argmax semantics).  Replaces the
 * temperature-0 branch of _sample_kernel (kavor/layers/sampler.py:7-45).
 * The workspace is optional (NULL allowed): with at least
 * kvp_argmax_workspace_bytes(num_rows) bytes (8-byte aligned, no initialisation needed),
 * batches of fewer than 192 rows split each row over several workgroups, which fills
 * the GPU (e.g. 9.6 -> 5.3 us for one 151936-wide row); without it every row is scanned
 * by one workgroup.  The result is the same either way.
 */
size_t kvp_argmax_workspace_bytes(int32_t num_rows);
int kvp_argmax_bf16(const void* logits, int64_t row_stride, int32_t num_rows, int32_t vocab,
                    int64_t* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sampling: for each row r with temperatures[r] > 0, out[r] = argmax_i of
 * logits[r, i] / temperatures[r] + g, g = -log(-log(u)) (Gumbel-max: a sample of
 * softmax(logits / T)); other rows (T <= 0 or NaN) take kvp_argmax_bf16's greedy index.
 * u is the reference sampler's noise stream: Triton's tl.rand(seed, i + r * vocab), the
 * first word of Philox4x32-10 for counter (i + r * vocab mod 2^32, 0, 0, 0) and the
 * sign-extended *seed as key, scaled to [0, 1).  *seed is read on the device, so a
 * captured graph draws new noise when the caller advances it between replays (the
 * reference's Sampler adds 1 before every call).  temperatures: num_rows fp32.  Ties
 * keep the first index; a NaN score counts as largest.  Replaces _sample_kernel and
 * Sampler.forward's launch (kavor/layers/sampler.py:7-66).  Workspace as for
 * kvp_argmax_bf16.
 */
int kvp_sample_bf16(const void* logits, int64_t row_stride, int32_t num_rows, int32_t vocab,
                    const float* temperatures, const int32_t* seed, int64_t* out,
                    void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAVOR_AMD_KVPATH_H */
