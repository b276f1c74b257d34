/*
 * femto_attn.h -- C ABI of libfemto_attn.so, the MI355X (gfx950) attention
 * hot path of FemtoVLLM (fishAndShrimp/nano-vllm-practice).
 *
 * Every entry point takes raw device pointers, element strides and sizes,
 * launches hand-written HIP kernels on the given stream (a hipStream_t
 * passed as void*, NULL = the null stream) and returns without
 * synchronising.  No entry point allocates device memory: outputs and the
 * decode workspace belong to the caller.  Inputs, including the KV pools,
 * are read-only.
 *
 * Return value: FEMTO_OK, or an error code with a message available from
 * femto_attn_last_error() (thread-local, valid until the next call on the
 * same thread).
 *
 * Layouts (all strides in elements, innermost dimension contiguous):
 *   paged pool  (num_blocks, n_kv_heads, block_size = 16, head_dim <= 128)
 *   block table (num_seqs, num_pages_per_seq) int32, -1 padded
 *   decode q/out  (n_heads, num_seqs, head_dim)
 *   prefill q/out (n_heads, num_tokens, head_dim), sequences by cu_seqlens
 *   dense q/out (batch, n_heads, q_len, head_dim), k/v (batch, n_kv_heads, kv_len, head_dim)
 */
#ifndef FEMTO_ATTN_H_
#define FEMTO_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum femto_status {
    FEMTO_OK = 0,
    FEMTO_ERR_INVALID = 1,     /* shape / stride / value check failed     */
    FEMTO_ERR_UNSUPPORTED = 2, /* dtype or size this library does not run */
    FEMTO_ERR_HIP = 3          /* HIP runtime error from a launch         */
};

enum femto_dtype { FEMTO_F32 = 0, FEMTO_F16 = 1, FEMTO_BF16 = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* femto_attn_last_error(void);

/* Compile-time constants the reference exports as _C attributes
 * (csrc/bindings.cpp:62-66 <- csrc/utils/constants.cuh:8, 39, 75):
 * kMaxKVLenNonSplit = 8192, kKVLenPerPage = 16, kDimHead = 128. */
int femto_attn_max_kv_len_non_split(void);
int femto_attn_kv_len_per_page(void);
int femto_attn_dim_head(void);

/* Bytes of workspace femto_paged_attention_gemv needs for these sizes when
 * it runs split (max_kv_len above the one-launch limit below).  It holds the
 * per-split partial softmax states between the split kernel and the merge
 * kernel of one call; no initialisation is needed.  Calls that may overlap
 * (other streams) must not share a workspace. */
size_t femto_paged_attention_gemv_workspace_size(int num_seqs, int n_heads, int max_kv_len);

/* Decode calls with max_kv_len at most this limit (default 1024 keys) run as
 * one kernel launch (a workgroup per sequence and KV head group) and use no
 * workspace; longer ones run the split kernel and the merge kernel.  Sets the
 * limit for the process (-1: always split) and returns the previous one.
 * No counterpart in the reference (whose decode is always one launch,
 * csrc/paged_attention/paged_attention_gemv.cu:280-300); it exists for tests
 * and tuning. */
int femto_attn_set_decode_single_max_kv(int max_kv_len);

/* Paged decode attention: one query token per sequence attends to all
 * kv_lens[b] keys of its block table; GQA kv head = h / (n_heads / n_kv_heads).
 * Replaces PagedAttentionGemvCuda (csrc/paged_attention/paged_attention_gemv.cu:223-308),
 * bound as _C.PagedAttentionGemvCuda (csrc/bindings.cpp:52-59, 94-97) and
 * called by femtovllm.ops.paged_attention_gemv (femtovllm/ops/__init__.py:82-107).
 * dtype: F32, F16 or BF16.  head_dim <= 128 (the reference's TORCH_CHECK_LE,
 * paged_attention_gemv.cu:256-257) in whole 16-byte chunks; scale 1/sqrt(head_dim).
 * kv_len == 0 yields a zero row, as in the reference.
 * workspace may be NULL (0 bytes) when max_kv_len is within the one-launch
 * limit of femto_attn_set_decode_single_max_kv. */
int femto_paged_attention_gemv(
    int dtype,
    const void* q, int64_t q_stride_head, int64_t q_stride_seq,
    void* out, int64_t out_stride_head, int64_t out_stride_seq,
    const void* k_pool, const void* v_pool,
    int64_t num_blocks, int n_kv_heads, int block_size, int head_dim,
    int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
    const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
    const int32_t* kv_lens, int num_seqs, int n_heads, int max_kv_len,
    void* workspace, size_t workspace_bytes,
    void* stream);

/* femto_paged_attention_gemv without a workspace argument: the partial
 * softmax states live in a 64 MiB device array of the library (one per GPU,
 * held until the process ends), so the call allocates nothing and can be
 * made where hipMalloc cannot (under HIP graph capture, in serving loops
 * that must not allocate).  No counterpart in the reference; it exists for
 * those callers.  Limit: two partial states of 130 floats per (sequence,
 * query head) must fit, i.e. num_seqs * n_heads up to about 64,500 (e.g. 2048
 * sequences x 32 heads); larger calls fail with FEMTO_ERR_INVALID.  When the default
 * split does not fit the array, sequences are cut into fewer, longer slices
 * (same results within rounding; bit-identical where the split is the
 * same).  All calls on one GPU share the array: calls that may overlap on
 * one GPU (different streams or threads) race and must be serialised by the
 * caller.  The first call on a device looks up the array's device address and
 * the CU count (hipGetSymbolAddress, hipDeviceGetAttribute): make it outside
 * graph capture; later calls only launch kernels and may be captured.  Every
 * process that loads the library reserves the 64 MiB on each GPU it uses,
 * whether or not it calls this entry point. */
int femto_paged_attention_gemv_noalloc(
    int dtype,
    const void* q, int64_t q_stride_head, int64_t q_stride_seq,
    void* out, int64_t out_stride_head, int64_t out_stride_seq,
    const void* k_pool, const void* v_pool,
    int64_t num_blocks, int n_kv_heads, int block_size, int head_dim,
    int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
    const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
    const int32_t* kv_lens, int num_seqs, int n_heads, int max_kv_len,
    void* stream);

/* Paged chunked / varlen / causal prefill attention on bf16 or f16 MFMA:
 * token t of sequence b (cu_seqlens[b] <= t < cu_seqlens[b+1]) sees key j
 * iff j < kv_lens[b] and j <= positions[t].
 * Replaces PagedAttentionGemmCuda (csrc/paged_attention/paged_attention_gemm.cu:304-395)
 * and paged_attention_gemm_triton
 * (femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:165-235),
 * bound as _C.PagedAttentionGemmCuda (csrc/bindings.cpp:41-50, 90-93) and
 * called by femtovllm.ops.paged_attention_gemm (femtovllm/ops/__init__.py:110-156).
 * dtype: F16 or BF16 (the reference kernels reject F32 too).  head_dim <=
 * 128 as the reference checks (paged_attention_gemm.cu:347-348), a multiple
 * of 16 (smaller ones run at the speed of 128); scale 1/sqrt(head_dim).  A
 * row with no visible key (kv_len == 0) is NaN, as in the reference.
 * max_q_len: the longest sequence's token count, as the reference binding
 * takes it; it only bounds how many sequences may have exactly one token.
 * workspace may be NULL.  With a workspace of at least
 * femto_paged_attention_gemm_workspace_size() bytes (256-byte aligned; its
 * first femto_paged_attention_gemm_split_bytes() bytes, the key-split
 * counters, zero-filled before the first use, and every call leaves them
 * zero-filled):
 *  - the query tiles of sequences much longer than the average are split
 *    over their keys and merged within the launch, so a few long sequences
 *    do not set the length of the call;
 *  - when num_seqs, num_tokens and max_q_len allow sequences of one query
 *    token (decode rows of a mixed batch), those rows run on the decode
 *    kernel's wave workers (the rest of the workspace holds their partial
 *    states) and the MFMA tiles skip them; the workers share the tiles'
 *    launch (a separate decode launch first when n_heads / n_kv_heads is a
 *    multiple of 8) and a small merge launch follows.  Without a workspace
 *    the MFMA kernel computes every row.
 * Every launch goes on `stream`.  Calls that may overlap (other streams)
 * must not share a workspace. */
int femto_paged_attention_gemm(
    int dtype,
    const void* q, int64_t q_stride_head, int64_t q_stride_token,
    void* out, int64_t out_stride_head, int64_t out_stride_token,
    const void* k_pool, const void* v_pool,
    int64_t num_blocks, int n_kv_heads, int block_size, int head_dim,
    int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
    const int32_t* cu_seqlens, int num_seqs, int num_tokens, int max_q_len, int n_heads,
    const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
    const int32_t* kv_lens, const int32_t* positions,
    void* workspace, size_t workspace_bytes,
    void* stream);

/* Bytes of the optional workspace of femto_paged_attention_gemm: the
 * key-split part (one counter and one 66 KiB partial slot per workgroup the
 * current device holds at once, 2 per CU, independent of the batch) plus,
 * when the sizes allow one-token sequences, the decode rows' partial states
 * (num_seqs x n_heads x slots of 130 floats, slots set by the table width
 * num_pages_per_seq); 0 for an empty call or without a device.  No
 * counterpart in the reference, whose prefill kernels take no workspace. */
size_t femto_paged_attention_gemm_workspace_size(int num_seqs, int num_tokens, int max_q_len, int n_heads,
                                                 int n_kv_heads, int num_pages_per_seq);

/* Leading bytes of that workspace that must be zero-filled before its first
 * use: the key-split counters (the partial slots behind them and the
 * decode-row part need no initialisation).  No counterpart in the
 * reference. */
size_t femto_paged_attention_gemm_split_bytes(void);

/* KV-cache write: scatter new K/V rows into the paged pools, bit-exact.
 * k, v: (num_tokens, n_kv_heads, head_dim), element strides per token and
 * per head (head_dim contiguous, rows 16-byte aligned).  Pools as above.
 * Sequence b's tokens are k[cu_seqlens[b] .. cu_seqlens[b+1]) at logical
 * positions positions[cu_seqlens[b]] + 0, 1, ...; position p goes to block
 * kv_page_tables[b][p / 16], row p % 16.  cu_seqlens == NULL means one token
 * per sequence (decode: num_tokens == num_seqs, token b at positions[b]).
 * max_q_len: the longest sequence's token count (tokens beyond it are not
 * written).  Writing stops, per sequence, at the first table column from
 * positions[q_begin] / 16 on that holds -1, a block id outside the pool or
 * lies past num_pages_per_seq.
 * Replaces the per-sequence slicing loops that write the cache before the
 * attention ops in the reference (femtovllm/models/qwen/qwen3.py:240-264 for
 * decode, 322-366 for prefill; "TODO use kernel" at line 240).
 * dtype: F32, F16 or BF16 (a byte copy; head_dim * element size a multiple
 * of 16). */
int femto_kv_cache_write(
    int dtype,
    const void* k, int64_t k_stride_token, int64_t k_stride_head,
    const void* v, int64_t v_stride_token, int64_t v_stride_head,
    void* k_pool, void* v_pool,
    int64_t num_blocks, int n_kv_heads, int block_size, int head_dim,
    int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
    const int32_t* cu_seqlens, int num_seqs, int num_tokens, int max_q_len,
    const int32_t* positions, const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
    void* stream);

/* Fused attention prologue: per-head RMSNorm of q and k (weights q_weight,
 * k_weight of head_dim elements, eps), rotary embedding of both at each
 * token's position (cos/sin: fp32 tables (rope_rows, head_dim) with row
 * stride rope_stride, as QwenRotaryEmbedding builds them), rotated q to
 * q_out (may alias q), rotated k and raw v into the pools by the rule of
 * femto_kv_cache_write (same cu_seqlens / positions / table arguments).
 * Computes in fp32 and rounds each output once; a position outside the
 * tables yields NaN rows.  head_dim must be 128.
 * Replaces q_norm / k_norm / rotary_embd and the cache-write loops of the
 * reference's attention layer (femtovllm/models/qwen/qwen3.py:230-264 for
 * decode, 312-366 for prefill; RMSNorm qwen3.py:181-183, RoPE 17-138),
 * which run as separate operators before the attention ops. */
int femto_qk_norm_rope_cache_write(
    int dtype,
    const void* q, int64_t q_stride_token, int64_t q_stride_head,
    const void* k, int64_t k_stride_token, int64_t k_stride_head,
    const void* v, int64_t v_stride_token, int64_t v_stride_head,
    void* q_out, int64_t q_out_stride_token, int64_t q_out_stride_head,
    const void* q_weight, const void* k_weight, float eps,
    const float* cos, const float* sin, int64_t rope_stride, int rope_rows,
    void* k_pool, void* v_pool,
    int64_t num_blocks, int n_heads, int n_kv_heads, int block_size, int head_dim,
    int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
    const int32_t* cu_seqlens, int num_seqs, int num_tokens, int max_q_len,
    const int32_t* positions, const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
    void* stream);

/* Varlen attention metadata built on the device, by the rules of the
 * reference's ModelRunner (femtovllm/engine/model_runner.py:187-202 prefill,
 * 283-293 decode, 46-72 block-table padding), which builds them with Python
 * loops and one host-to-device copy per tensor.  Inputs (device, int32):
 * num_computed[b] (= pos), num_tokens[b] (= n), the block tables in CSR form
 * (block_offsets (num_seqs+1), block_ids).  Outputs: positions (sum n) =
 * pos .. pos+n-1 per sequence, cu_seqlens / cu_q_tiles (num_seqs+1) prefix
 * sums of n / ceil(n / q_tile_size), q_tile_to_seq_idx, kv_lens = pos + n,
 * block_tables (num_seqs, table_width) padded with -1.  max_q_len: the
 * largest n (table_width: the longest table). */
int femto_build_varlen_metadata(
    int num_seqs, const int32_t* num_computed, const int32_t* num_tokens,
    const int32_t* block_offsets, const int32_t* block_ids, int table_width,
    int q_tile_size, int max_q_len,
    int32_t* positions, int32_t* cu_seqlens, int32_t* cu_q_tiles, int32_t* q_tile_to_seq_idx,
    int32_t* kv_lens, int32_t* block_tables,
    void* stream);

/* Dense non-causal GQA flash attention, q (B, H, Tq, D), k/v (B, KVH, Tkv, D).
 * Replaces FlashAttentionWarpCuda (csrc/flash_attention/flash_attention_warp.cu:301-376),
 * bound as _C.FlashAttentionWarpCuda (csrc/bindings.cpp:35-39, 86-89).
 * dtype: F16 or BF16. */
int femto_flash_attention(
    int dtype,
    const void* q, int64_t q_stride_batch, int64_t q_stride_head, int64_t q_stride_token,
    const void* k, int64_t k_stride_batch, int64_t k_stride_head, int64_t k_stride_token,
    const void* v, int64_t v_stride_batch, int64_t v_stride_head, int64_t v_stride_token,
    void* out, int64_t out_stride_batch, int64_t out_stride_head, int64_t out_stride_token,
    int batch, int n_heads, int n_kv_heads, int q_len, int kv_len, int head_dim,
    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FEMTO_ATTN_H_ */
