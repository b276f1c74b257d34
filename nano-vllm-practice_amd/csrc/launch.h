// Kernel argument blocks and launchers (host side of the HIP kernels).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace femto {

enum { kDtypeF32 = 0, kDtypeF16 = 1, kDtypeBF16 = 2 };

struct DecodeArgs {
    const void* q;
    int64_t q_stride_head, q_stride_seq;
    void* out;
    int64_t out_stride_head, out_stride_seq;
    const void* k_pool;
    const void* v_pool;
    int64_t num_blocks;
    int64_t pool_stride_block, pool_stride_head, pool_stride_row;
    const int32_t* tables;
    int64_t table_stride;
    int num_pages_per_seq;
    const int32_t* kv_lens;
    int num_seqs;
    int n_heads, n_rep, head_groups;
    int grid_heads;       // n_heads / nrep_tile: KV head groups
    int waves_per_group;  // set by the launcher from the resident wave count
    int min_chunk_pages;  // lower bound on a wave's slice length
    int max_slots;        // partial slots per (sequence, head)
    int head_dim;         // 128, or a smaller multiple of 16 bytes (decode calls only)
    int single_waves;     // one-launch kernel: waves per workgroup (4, or 8 with one query head per wave)
    float scale_log2;
    float* part_acc;  // [num_seqs][n_heads][max_slots][128]
    float* part_ml;   // [num_seqs][n_heads][max_slots][2]
    int* seq_slots;   // [num_seqs] partial slots written for the sequence
    // Decode rows of a varlen prefill call (both null for a decode call):
    // sequence b takes part iff it has exactly one query token, that token
    // is row cu_seqlens[b] of q and out, and it sees keys
    // j < min(kv_lens[b], positions[row] + 1).
    const int32_t* cu_seqlens;
    const int32_t* positions;
};

// Compute units of the current device, queried once per device (safe to call
// from several host threads).
hipError_t device_cu_count(int& cus);

// Work split of a decode call.
struct DecodePlan {
    int nrep_tile;        // query heads per wave
    int min_chunk_pages;  // pages
    int max_slots;
};
DecodePlan plan_paged_decode(int n_heads, int n_kv_heads, int max_kv_len, int dtype);
size_t decode_workspace_bytes(int num_seqs, int n_heads, int max_slots);

// single: the one-launch kernel (decode calls only, no workspace), else the
// split workers and the merge kernel.
hipError_t launch_paged_decode(int dtype, const DecodeArgs& a, int nrep_tile, int num_seqs, bool single,
                               hipStream_t st);
// Decode workers of a fused prefill launch: workgroups needed (sets
// a.waves_per_group; 0 on a device error), and the merge that follows.
int decode_worker_blocks(DecodeArgs& a);
hipError_t launch_paged_decode_merge(int dtype, const DecodeArgs& a, int num_seqs, hipStream_t st);

struct PrefillArgs {
    const void* q;
    int64_t q_stride_batch, q_stride_head, q_stride_token;
    void* out;
    int64_t out_stride_batch, out_stride_head, out_stride_token;
    const void* k;
    const void* v;
    // paged: block / kv head / row strides of the pools; dense: batch /
    // kv head / token strides of k and v.
    int64_t k_stride0, k_stride1, k_stride2;
    int64_t v_stride0, v_stride1, v_stride2;
    int64_t num_blocks;
    const int32_t* cu_seqlens;  // paged only
    const int32_t* tables;      // paged only
    int64_t table_stride;
    int num_pages_per_seq;
    const int32_t* kv_lens;    // paged only
    const int32_t* positions;  // paged only (causal)
    int num_seqs;              // paged: sequences; dense: batch
    int q_len, kv_len;         // dense only
    int n_heads, n_kv_heads, n_rep, head_groups;
    int tiles_per_group;  // upper bound on workgroups per (kv head, head group)
    int total_work;       // tiles_per_group * n_kv_heads * head_groups (grid size)
    int head_dim;         // 128; paged calls also a smaller multiple of 16
    float scale_log2;
    // Key split of long query tiles (paged only; part == nullptr: none).
    float* part;          // one partial slot of kPartSlotBytes per resident workgroup
    int* counters;        // one arrival counter per resident workgroup
    int items_per_group;  // upper bound on query tiles per (kv head, head group)
    int resident;         // workgroups the GPU holds at once
    int skip_decode_rows; // sequences of one query token are left to the decode workers
    // Decode workers in the same launch (paged only): the first decode_blocks
    // workgroups run the decode kernel's waves over `dec` (one-token
    // sequences), the rest the MFMA tiles; 0: none.
    int decode_blocks;
    DecodeArgs dec;
};

// Key split: at most kMaxPieces pieces per query tile, each leaving a
// partial (m, l, O) slot: 4 waves x 64 lanes x (64 accumulators + m, l).
constexpr int kMaxPieces = 8;
constexpr int kPartSlotBytes = 4 * 64 * 64 * 4 + 4 * 64 * 8;
hipError_t prefill_resident_workgroups(int& resident);
size_t prefill_counter_bytes(int resident);
size_t prefill_workspace_bytes(int resident);

// KV-cache write (kv_cache_write.hip).
struct CacheWriteArgs {
    const void* k;  // (tokens, n_kv_heads, head_dim), any token / head strides
    const void* v;
    int64_t k_stride_token, k_stride_head;
    int64_t v_stride_token, v_stride_head;
    void* k_pool;  // (num_blocks, n_kv_heads, 16, head_dim), both pools with the same strides
    void* v_pool;
    int64_t num_blocks;
    int64_t pool_stride_block, pool_stride_head, pool_stride_row;
    const int32_t* cu_seqlens;  // null: one token per sequence (decode)
    const int32_t* positions;   // logical position of each sequence's first token at positions[q_begin]
    const int32_t* tables;
    int64_t table_stride;
    int num_pages_per_seq;
    int num_seqs;
    int n_kv_heads;
    int row_chunks;  // head_dim * elem_bytes / 16
    int elem_bytes;
};

hipError_t launch_kv_cache_write(const CacheWriteArgs& a, int max_q_len, hipStream_t st);

// Fused QK-norm + RoPE + KV-cache write (qk_norm_rope.hip).  cw describes
// the k/v sources, the pools and the placement exactly as for
// kv_cache_write; cw.positions[q_begin] places each sequence, and
// positions_rope[t] (the same array) is each token's rotary position.
struct PrologueArgs {
    CacheWriteArgs cw;
    const void* q;  // (tokens, n_heads, 128)
    int64_t q_stride_token, q_stride_head;
    void* q_out;    // (tokens, n_heads, 128), may alias q
    int64_t q_out_stride_token, q_out_stride_head;
    const void* q_weight;  // (128,) RMSNorm weights, storage type
    const void* k_weight;
    float eps;
    const float* cos;  // (rope_rows, >= 128) fp32
    const float* sin;
    int64_t rope_stride;
    int rope_rows;
    const int32_t* positions_rope;
    int n_heads;
};

hipError_t launch_qk_norm_rope(int dtype, const PrologueArgs& a, int max_q_len, hipStream_t st);

// Varlen metadata build (varlen_metadata.hip).
struct MetadataArgs {
    const int32_t* num_computed;   // (num_seqs,)
    const int32_t* num_tokens;     // (num_seqs,)
    const int32_t* block_offsets;  // (num_seqs + 1,) CSR offsets into block_ids
    const int32_t* block_ids;
    int num_seqs, table_width, q_tile_size;
    int32_t* positions;          // (sum num_tokens,)
    int32_t* cu_seqlens;         // (num_seqs + 1,)
    int32_t* cu_q_tiles;         // (num_seqs + 1,)
    int32_t* q_tile_to_seq_idx;  // (sum ceil(num_tokens / q_tile_size),)
    int32_t* kv_lens;            // (num_seqs,)
    int32_t* block_tables;       // (num_seqs, table_width), -1 padded
};

hipError_t launch_varlen_metadata(const MetadataArgs& a, int max_q_len, hipStream_t st);

// decode_rows_max: upper bound on the one-token sequences when
// a.skip_decode_rows is set (0 otherwise).  With a.decode_blocks > 0 the
// decode workers run in the same launch (a.dec's head groups must hold
// prefill_group(n_rep) heads each) and the merge follows on `st`.
hipError_t launch_paged_prefill(int dtype, PrefillArgs a, int num_tokens, int decode_rows_max, hipStream_t st);
int prefill_group(int n_rep);
hipError_t launch_dense_attention(int dtype, PrefillArgs a, hipStream_t st);

}  // namespace femto
