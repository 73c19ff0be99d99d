/*
 * glm53.h -- C ABI of libglm53_hip.so, the MI355X (gfx950) kernels behind
 * the GLM-5.3 decode hot path.
 *
 * Every entry point takes device pointers, element or byte strides and a
 * HIP stream (hipStream_t passed as void*), enqueues its kernels on that
 * stream and returns 0 on success.  Nothing here allocates device memory,
 * synchronises the stream or reads device data on the host, so every call
 * may be captured into a HIP graph.  A negative return is an argument error
 * (see glm53_error_string); a positive return is the hipError_t of a failed
 * launch.  No torch or HIP types appear in the signatures.
 */
#ifndef GLM53_H_
#define GLM53_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLM53_ABI_VERSION 3

/* Argument errors (negative return codes). */
#define GLM53_ERR_NULL_POINTER   (-1)
#define GLM53_ERR_BAD_SHAPE      (-2)
#define GLM53_ERR_MISALIGNED     (-3)
#define GLM53_ERR_WORKSPACE      (-4)
#define GLM53_ERR_BAD_DTYPE      (-5)
#define GLM53_ERR_SCRATCH_LIMIT  (-6)   /* beyond glm53_sparse_mla_noalloc's static scratch */

int glm53_abi_version(void);
const char* glm53_error_string(int code);

/*
 * Per-token symmetric INT8 latent writer.
 * Replaces the launch of _store_int8 in store_int8 (kernels/titan_kv.py:23-28;
 * kernel body kernels/titan_kv.py:7-21).
 *
 * For each i in [0, n_slots): slot = slots[i]; if slot >= 0 the 528-byte row
 * at cache + (slot / block_size) * cache_stride_block
 *             + (slot % block_size) * cache_stride_slot
 * receives 512 int8 values q = clamp(rint(x / s), -127, 127) with
 * s = max(max|x| / 127, 1e-12) in IEEE fp32, then s as fp32 at byte 512 and
 * zeros in bytes 516..527.  x is bf16 row i (x + i * x_row_stride elements,
 * 512 contiguous values).  A negative slot leaves the cache untouched, and so
 * does a slot >= capacity (the number of slots the cache holds; the
 * reference leaves out-of-range positive slots undefined).
 *   slots_is_i64: 1 for int64 slots, 0 for int32 slots.
 *   cache strides are in bytes.
 */
int glm53_store_int8(const void* x, int64_t x_row_stride,
                     void* cache, int64_t cache_stride_block,
                     int64_t cache_stride_slot, int64_t block_size,
                     int64_t capacity, const void* slots, int slots_is_i64,
                     int64_t n_slots, void* stream);

/*
 * Sparse NoPE MLA attention over top-k indices into the 528-byte INT8 cache.
 * Replaces the kernel launches of triton_mla_sparse_attention
 * (kernels/titan_mla.py:500-581: _sparse_mla_kernel_final,
 * _sparse_mla_kernel_split and _sparse_mla_merge_kernel).
 *
 *   q        bf16 [num_tokens, num_heads, 512], strides sq_t, sq_h (elements),
 *            last dim contiguous, 16-byte aligned rows; num_tokens at most
 *            65535 (the grid's y dimension) in this and every other
 *            attention entry point, else GLM53_ERR_BAD_SHAPE.
 *   kv       528-byte rows, row r at kv + r * skv_t bytes (skv_t % 16 == 0),
 *            seq_kv rows; only the first 528 bytes of a row are read.
 *   indices  int32 [num_tokens, topk] with row stride si_t (elements); an
 *            index outside [0, seq_kv) is masked out.
 *   sm_scale softmax scale; logits are q.k * scale_j * fp32(sm_scale*log2 e)
 *            in base 2, as the reference computes them.
 *   num_splits  1..1024; the top-k axis is cut into num_splits slices of
 *            ceil(topk / num_splits) indices whose partial results are merged
 *            by log-sum-exp.  1 = single pass.
 *   workspace   device scratch of glm53_sparse_mla_workspace_bytes(...)
 *            bytes (unused when num_splits == 1; may then be NULL).
 *   out      bf16 [num_tokens, num_heads, 512], strides so_t, so_h.
 * A query whose indices are all masked produces exactly 0.
 */
int64_t glm53_sparse_mla_workspace_bytes(int64_t num_tokens, int64_t num_heads,
                                         int64_t num_splits);
int glm53_sparse_mla(const void* q, int64_t sq_t, int64_t sq_h,
                     const void* kv, int64_t skv_t, int64_t seq_kv,
                     const int32_t* indices, int64_t si_t,
                     int64_t num_tokens, int64_t num_heads, int64_t topk,
                     double sm_scale, int64_t num_splits,
                     void* workspace, int64_t workspace_bytes,
                     void* out, int64_t so_t, int64_t so_h,
                     void* stream);

/*
 * glm53_sparse_mla without a workspace argument and without any allocation:
 * the split partials go to a static device array of the library (one per
 * GPU, held until the process ends), so the call suits callers that cannot
 * allocate device memory (code under HIP graph capture that must not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  Same arguments, kernels and output as
 * glm53_sparse_mla; limit: num_tokens * num_splits * (num_heads rounded up
 * to 16) <= GLM53_NOALLOC_MAX_PARTIAL_ROWS when num_splits > 1, else
 * GLM53_ERR_SCRATCH_LIMIT (nothing launched).  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams) race.
 * Nothing in it needs clearing: a call writes every partial row it reads.
 */
#define GLM53_NOALLOC_MAX_PARTIAL_ROWS 8192
int glm53_sparse_mla_noalloc(const void* q, int64_t sq_t, int64_t sq_h,
                             const void* kv, int64_t skv_t, int64_t seq_kv,
                             const int32_t* indices, int64_t si_t,
                             int64_t num_tokens, int64_t num_heads, int64_t topk,
                             double sm_scale, int64_t num_splits,
                             void* out, int64_t so_t, int64_t so_h,
                             void* stream);

/*
 * Request-relative indices.  The reference's vLLM adapter converts the
 * indexer's request-relative token positions to flat cache rows with
 * vLLM's triton_convert_req_index_to_global_index and then calls the
 * attention (integration/titan_backend.py:48-54).  Mapping of one position
 * p of query token t (req = req_id[t]):
 *   p < 0, req outside [0, num_reqs), or p / block_size >= max_blocks -> -1;
 *   otherwise block_table[req * bt_stride + p / block_size] * page_rows
 *             + p % block_size   (32-bit wrapping arithmetic)
 * page_rows (>= block_size) is the row count of one physical page in the
 * flat row view (vLLM's BLOCK_STRIDE_ROWS; block_size for unpadded pages).
 * glm53_convert_req_index writes the mapped rows (int32 [num_tokens, topk],
 * row stride so_t) -- the conversion alone.
 */
int glm53_convert_req_index(const int32_t* req_id, const int32_t* block_table,
                            int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                            const int32_t* indices, int64_t si_t, int32_t* out,
                            int64_t so_t, int64_t num_tokens, int64_t topk,
                            int64_t block_size, int64_t page_rows, void* stream);

/*
 * glm53_sparse_mla with request-relative indices resolved inside the
 * attention's index load (one launch fewer per decode step than converting
 * first; the same output whenever the flat row view exists).  The cache is
 * paged: kv_pages is page 0, physical page b starts b * page_bytes bytes
 * later and holds block_size rows row_bytes apart (page_bytes and row_bytes
 * multiples of 16, row_bytes >= 528; the page stride may be padded to any
 * alignment, it need not be a whole number of rows).  Position p of token t
 * reads row p % block_size of page block_table[req_id[t], p / block_size];
 * it is masked when p < 0, the request id or block is outside the table, or
 * the table entry is not in [0, num_blocks).  num_blocks * page_bytes must
 * stay below 32 GiB.
 */
int glm53_sparse_mla_paged(const void* q, int64_t sq_t, int64_t sq_h,
                           const void* kv_pages, int64_t page_bytes, int64_t row_bytes,
                           int64_t num_blocks,
                           const int32_t* req_indices, int64_t si_t,
                           const int32_t* req_id, const int32_t* block_table,
                           int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                           int64_t block_size,
                           int64_t num_tokens, int64_t num_heads, int64_t topk,
                           double sm_scale, int64_t num_splits,
                           void* workspace, int64_t workspace_bytes,
                           void* out, int64_t so_t, int64_t so_h,
                           void* stream);

/*
 * Pool expansion, the last step of the sparse indexer: it selects the top-k
 * pools of pool_size consecutive tokens and expands them to token positions
 * (model: tests/verify_indexer_sharding.py:72-79).  Row t, slot k:
 *   k < num_pools * pool_size:  pool_ids[t][k / pool_size] * pool_size
 *                               + k % pool_size, or -1 for a negative id;
 *   next pool_size - 1 slots (seq_lens given): the tail tokens
 *                               seq_lens[t] / pool_size * pool_size + j for
 *                               j < seq_lens[t] % pool_size, else -1;
 *   later slots:                -1.
 * glm53_expand_pools writes slots [0, out_cols) (int32, row stride so_t);
 * pool ids are int32 or int64 (ids_is_i64), row stride sp_t elements;
 * seq_lens may be NULL (no tail slots).  glm53_sparse_mla_pooled is
 * glm53_sparse_mla_paged with each index slot computed this way inside the
 * attention's index load (int32 pool ids): the indexer's pool ids go
 * straight to the attention.
 */
int glm53_expand_pools(const void* pool_ids, int ids_is_i64, int64_t sp_t,
                       int64_t num_pools, const int32_t* seq_lens, int64_t pool_size,
                       int32_t* out, int64_t so_t, int64_t num_rows, int64_t out_cols,
                       void* stream);
int glm53_sparse_mla_pooled(const void* q, int64_t sq_t, int64_t sq_h,
                            const void* kv_pages, int64_t page_bytes, int64_t row_bytes,
                            int64_t num_blocks,
                            const int32_t* pool_ids, int64_t sp_t, int64_t num_pools,
                            const int32_t* seq_lens, int64_t pool_size,
                            const int32_t* req_id, const int32_t* block_table,
                            int64_t num_reqs, int64_t bt_stride, int64_t max_blocks,
                            int64_t block_size,
                            int64_t num_tokens, int64_t num_heads, int64_t topk,
                            double sm_scale, int64_t num_splits,
                            void* workspace, int64_t workspace_bytes,
                            void* out, int64_t so_t, int64_t so_h,
                            void* stream);

/*
 * The two stages of glm53_sparse_mla, exposed for callers that merge split
 * results themselves (for example after gathering one token's splits from
 * several devices).  Same stages as the reference's _sparse_mla_kernel_split
 * and _sparse_mla_merge_kernel (kernels/titan_mla.py:258-429).
 *
 * Partials layout (fp32), rows = num_tokens * num_splits * Hp with
 * Hp = num_heads rounded up to a multiple of 16, row r = (t * num_splits +
 * s) * Hp + h, head group hg = h / 16, c = h % 16:
 *   part[rows * 512]  normalised split output acc / l  (0 for an empty split),
 *                     in blocks of 16 heads x 512 latents per (t, s, hg) at
 *                     ((t * num_splits + s) * Hp / 16 + hg) * 8192 floats;
 *                     within a block, latent d of head c is float
 *                     ((8 * (d / 128) + d % 128 / 16) * 64 + 16 * (d % 16 / 4)
 *                     + c) * 4 + d % 4 (the MFMA accumulator order of the
 *                     kernels, so that each store instruction writes 1 KB)
 *   lse[rows]         (m + log2 l) * ln 2, natural-log LSE (-inf when empty)
 * glm53_sparse_mla_partials writes them for any num_splits >= 1;
 * glm53_sparse_mla_merge combines them into bf16 out with log-sum-exp
 * weights.  glm53_sparse_mla_partials_bytes gives the buffer size.
 */
int64_t glm53_sparse_mla_partials_bytes(int64_t num_tokens, int64_t num_heads,
                                        int64_t num_splits);
int glm53_sparse_mla_partials(const void* q, int64_t sq_t, int64_t sq_h,
                              const void* kv, int64_t skv_t, int64_t seq_kv,
                              const int32_t* indices, int64_t si_t,
                              int64_t num_tokens, int64_t num_heads, int64_t topk,
                              double sm_scale, int64_t num_splits,
                              void* partials, int64_t partials_bytes,
                              void* stream);
/*
 * Diagnostic, no counterpart in the reference: the memory chain of
 * glm53_sparse_mla_partials alone for decode splits (at most 256 indices per
 * split) -- the same grid, index loads, row gathers, scale loads and
 * partial/LSE stores, issued in the split kernel's order and all in flight
 * before any is used, with no arithmetic (the partials hold junk).  Its
 * time is the floor that the split kernel's conversions, products and
 * softmax add to; bench.py reports both.  Needs seq_kv >= 1 (masked keys
 * read row 0).
 */
int glm53_sparse_mla_gather_floor(const void* q, int64_t sq_t, int64_t sq_h,
                                  const void* kv, int64_t skv_t, int64_t seq_kv,
                                  const int32_t* indices, int64_t si_t,
                                  int64_t num_tokens, int64_t num_heads, int64_t topk,
                                  int64_t num_splits, void* partials, int64_t partials_bytes,
                                  void* stream);
int glm53_sparse_mla_merge(const void* partials, int64_t partials_bytes,
                           int64_t num_tokens, int64_t num_heads,
                           int64_t num_splits, void* out, int64_t so_t,
                           int64_t so_h, void* stream);

/*
 * Stable MoE route alignment for 1..8 tokens, top-8 routing, 288 experts,
 * block size 8, invalid routes ignored.
 * Replaces the launch of _align_small in titan_moe_align_small
 * (kernels/titan_moe_align.py:49-81; kernel body :12-46).
 *
 *   topk_ids  int32 or int64 (ids_is_i64) [num_routes], num_routes in [1, 64]
 *   sorted_ids  int32 [num_routes * 8]: flat route ids grouped by expert in
 *               ascending expert order, stable within an expert, each
 *               expert padded to a multiple of 8 with num_routes; the tail
 *               is num_routes as well.
 *   expert_ids  int32 [num_routes]: expert of each 8-block, then -1.
 *   num_tokens_post_padded  int32 [1]: sum over experts of ceil8(count).
 * Routes outside [0, 288) (compared at full 64-bit width) are dropped.
 */
int glm53_moe_align_small(const void* topk_ids, int ids_is_i64,
                          int64_t num_routes, int32_t* sorted_ids,
                          int32_t* expert_ids,
                          int32_t* num_tokens_post_padded, void* stream);

/*
 * W4A16 group-32 MoE expert GEMMs: the consumer of glm53_moe_align_small.
 * Replace the two moe_wna16_marlin_gemm launches, the activation and the
 * moe_sum of vLLM's fused Marlin MoE at the GLM-5.3 call site (the call
 * sequence profiles/sm74/titan_prefill/marlin.py:424-444, gated on
 * marlin.py:255-310: bf16 activations, uint4b8 weights with bf16 group-32
 * scales and no zero points, SiLU with clamp, router weight on the output;
 * the aligner's call site integration/patch_moe_align.py:17-44).
 *
 * With W = (q - 8) * s (q the unsigned 4-bit code, s the bf16 scale of its
 * 32-feature group) and route r = t * topk + j of token t with expert
 * e = topk_ids[t, j] and weight w = topk_weights[t, j]:
 *   c1[r] = bf16(x[t] . W13[e]^T)                         (2N values)
 *   c2[r] = bf16(silu(min(g, L)) * min(max(u, -L), L))    g = c1[r, :N], u = c1[r, N:]
 *   c3[r] = bf16(w * (c2[r] . W2[e]^T))                   (K values)
 *   out[t] = bf16(c3[t*topk] + ... + c3[t*topk + topk-1]) (fp32 sum in slot order)
 * Routes whose expert lies outside [0, num_experts) contribute 0.
 * L = clamp_limit (> 0; +inf for plain SiLU-and-multiply).
 *
 * Weights: checkpoint int32 [E][n_out][K/8] (word w of row n holds k = 8w+i
 * in bits 4i, the GPTQ / compressed-tensors packing) with bf16 scales
 * [E][n_out][K/32] are repacked once by glm53_moe_w4a16_repack into the
 * kernels' tile order (same sizes: int32 [E][n_out/16][K/128][64][4] and
 * bf16 [E][n_out/16][K/128][16][4]); W13 is [E][2N][K] (gate rows, then up
 * rows), W2 is [E][K][N].  K is a multiple of 128 and N of 16 for W13, N a
 * multiple of 128 for W2.
 */
/* Repack [E][n_out][k/8] int32 words (w_packed, 4-byte aligned) and their
 * bf16 scales [E][n_out][k/32] (w_scale) into the tile order at out
 * (16-byte aligned) and out_scale (8-byte aligned).  n_out % 16 == 0,
 * k % 128 == 0. */
int glm53_moe_w4a16_repack(const void* w_packed, const void* w_scale,
                           int64_t num_experts, int64_t n_out, int64_t k,
                           void* out, void* out_scale, void* stream);

/* c2 for every route of the aligner's blocks: one workgroup per (8-slot
 * block b with expert_ids[b] in [0, E), 16 intermediate columns); slots
 * holding num_routes are padding.  x bf16 [T][hidden], row stride sx
 * elements (16-byte aligned rows), hidden <= 4096; act bf16
 * [num_routes][n_inter]. */
int glm53_moe_w4a16_gate_up(const void* x, int64_t sx, const void* w13,
                            const void* s13, const int32_t* sorted_ids,
                            const int32_t* expert_ids, int64_t num_routes,
                            int64_t topk, int64_t num_experts,
                            int64_t n_inter, int64_t hidden,
                            float clamp_limit, void* act, void* stream);

/* out for every token: one workgroup per (16 output features, token), the
 * token's topk (<= 8) routes summed in slot order; n_inter <= 2048.  topk_ids int32 or int64
 * (ids_is_i64) [T][topk] with row stride sid_t; topk_weights fp32 [T][topk]
 * with row stride sw_t; out bf16 [T][hidden], row stride so. */
int glm53_moe_w4a16_down(const void* act, const void* w2, const void* s2,
                         const void* topk_ids, int ids_is_i64, int64_t sid_t,
                         const float* topk_weights, int64_t sw_t,
                         int64_t num_tokens, int64_t topk,
                         int64_t num_experts, int64_t n_inter,
                         int64_t hidden, void* out, int64_t so, void* stream);

/* Bytes of the workspace glm53_fused_moe_w4a16 needs (the c2 activations,
 * bf16 [num_tokens * topk][n_inter]). */
int64_t glm53_fused_moe_w4a16_workspace_bytes(int64_t num_tokens,
                                              int64_t topk, int64_t n_inter);

/* The whole layer for 1..8 tokens, top-8, 288 experts (the aligner's
 * contract); topk_ids and topk_weights contiguous [T][8].  Two launches: the
 * gate/up kernel derives each workgroup's aligner block (expert and slots,
 * the layout glm53_moe_align_small writes) from topk_ids itself, then the
 * down kernel. */
int glm53_fused_moe_w4a16(const void* x, int64_t sx, const void* w13,
                          const void* s13, const void* w2, const void* s2,
                          const void* topk_ids, int ids_is_i64,
                          const float* topk_weights, int64_t num_tokens,
                          int64_t topk, int64_t num_experts, int64_t n_inter,
                          int64_t hidden, float clamp_limit, void* workspace,
                          int64_t workspace_bytes, void* out, int64_t so,
                          void* stream);

/*
 * Sparse indexer decode scoring: FP8 paged MQA logits.
 * Replaces vLLM's fp8_paged_mqa_logits_triton as the reference's decode
 * indexer calls it (integration/patch_decode_indexer.py:34-44, pool-granular
 * context); semantics of DeepGEMM's fp8_paged_mqa_logits:
 *   logits[t, j] = sum_h weights[t, h] * max(0, s_j * (q[t, h, :] . k_j))
 * for j < context_lens[t]; -inf where block_table[t, j / block_size] is not
 * in [0, num_blocks); positions in [context_lens[t], max_len) are set to -inf
 * when clean_logits, else left untouched.
 *   q        fp8 E4M3 (OCP) [T][H][128], byte strides sq_t, sq_h (16-byte aligned)
 *   kv_cache pages of page_bytes bytes: block_size keys x 128 fp8 bytes, then
 *            block_size fp32 scales (the fused layout [num_blocks, block_size,
 *            1, 132]); key j of row t lives in page block_table[t, j / block_size]
 *   weights  fp32 [T][H] (row stride sw_t); H in {16, 32, 48, 64}
 *   logits   fp32 [T][max_len] (row stride sl_t)
 */
int glm53_fp8_paged_mqa_logits(const void* q, int64_t sq_t, int64_t sq_h,
                               const void* kv_cache, int64_t page_bytes,
                               int64_t block_size, int64_t num_blocks,
                               const float* weights, int64_t sw_t,
                               const int32_t* context_lens,
                               const int32_t* block_table, int64_t bt_stride,
                               int64_t max_blocks, int64_t num_tokens,
                               int64_t num_heads, int64_t head_dim,
                               int64_t max_len, int clean_logits,
                               float* logits, int64_t sl_t, void* stream);

/*
 * Top-k per row of the indexer logits: the top-512 pool selection whose pool
 * ids (topk_dst / pool_topk) the kpool expansion consumes
 * (integration/patch_indexer_sharding.py:58-79,
 * integration/patch_decode_indexer.py:64-72; vLLM's radix top-k): the k
 * largest of logits[r, 0 : lengths[r]] (lengths clamped to [0, max_len]; NaN
 * ranks lowest, ties by smaller position), written as positions in ascending
 * order; a row with fewer than k valid positions gets all of them, then -1.
 *   logits     fp32 [num_rows][max_len], row stride sl (rows 16-byte aligned load
 *              4 keys at a time, others one at a time)
 *   workspace  device scratch of glm53_indexer_topk_workspace_bytes(...) bytes
 *              (0 for rows of at most 4096 columns; may then be NULL); the
 *              size asked for num_rows rows serves every call with at most
 *              that many rows (same max_len and k)
 *   out        int32 [num_rows][k], row stride so
 */
int64_t glm53_indexer_topk_workspace_bytes(int64_t num_rows, int64_t max_len,
                                           int64_t k);
int glm53_indexer_topk(const float* logits, int64_t sl, const int32_t* lengths,
                       int64_t num_rows, int64_t max_len, int64_t k,
                       void* workspace, int64_t workspace_bytes,
                       int32_t* out, int64_t so, void* stream);

/*
 * Diagnostic, no counterpart in the reference: stream `bytes` (a multiple of
 * 16, both pointers 16-byte aligned) from src with 16-byte lane loads, the
 * ceilings that bench.py reads the bandwidth-bound kernels against.
 *   GLM53_PROBE_READ     plain loads, data folded and discarded (dst: one
 *                        16-byte sink, written only for one magic value)
 *   GLM53_PROBE_READ_NT  the same with non-temporal loads
 *   GLM53_PROBE_COPY_NT  copy src -> dst (bytes each) with non-temporal
 *                        loads and stores
 */
#define GLM53_PROBE_READ     0
#define GLM53_PROBE_READ_NT  1
#define GLM53_PROBE_COPY_NT  2
int glm53_stream_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GLM53_H_ */
