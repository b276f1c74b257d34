// KV-cache write: scatter the new K/V rows of a varlen batch into the
// paged pools (num_blocks, n_kv_heads, 16, head_dim).
//
// Semantics follow the per-sequence slicing loops that the reference runs
// before its attention ops (femtovllm/models/qwen/qwen3.py:240-264 for
// decode, 322-366 for prefill): the tokens of sequence b, k[q_begin ..
// q_end), go to logical positions p0, p0 + 1, ... with p0 =
// positions[q_begin]; position p lands in block tables[b][p / 16], row
// p % 16, all KV heads.  The reference walks the table from column p0 / 16
// and stops at the first -1, so a token is written only if every column
// from p0 / 16 up to its own holds a block id; here a column past the
// table width or a block id outside the pool stops the walk too (the
// reference would index out of bounds).  Rewriting a token whose block is
// shared (the scheduler's (L-1) re-run of a cached token) stores the same
// bytes again.  The copy is bit-exact for every element type.
//
// Work: workgroup (x, b) copies tokens q_begin + 4x .. + 3 of sequence b
// (they span at most two pages), then the same four tokens gridDim.x * 4
// further on, until the sequence ends.  Each thread moves 16-byte chunks; a
// token is 2 * n_kv_heads * head_dim * element_bytes / 16 chunks (256 for
// 8 bf16 heads of 128), so one pass of 256 threads x 4 chunks covers the
// four tokens.  The source rows depend only on cu_seqlens, so their loads
// are issued before the destination is looked up (positions, then the
// block table): the copy costs about three dependent memory round trips.
#include "common.h"
#include "launch.h"

namespace femto {

constexpr int kWriteTokens = 4;   // tokens per workgroup
constexpr int kWriteBatch = 8;    // chunks in flight per thread

__global__ __launch_bounds__(256) void kv_cache_write_kernel(CacheWriteArgs a) {
    __shared__ int s_stop, s_blk[2];
    const int b = blockIdx.y;
    int q_begin, q_end;
    if (a.cu_seqlens) {
        q_begin = a.cu_seqlens[b];
        q_end = a.cu_seqlens[b + 1];
    } else {  // decode: one token per sequence
        q_begin = b;
        q_end = b + 1;
    }
    // max_q_len only sizes the grid: a sequence longer than it is covered
    // by later rounds of the same workgroups (the loop condition is uniform
    // across the workgroup, so the barriers inside stay matched).
    for (int t0 = q_begin + (int)blockIdx.x * kWriteTokens; t0 < q_end; t0 += (int)gridDim.x * kWriteTokens) {
    const int t1 = min(q_end, t0 + kWriteTokens);

    const int cpr = a.row_chunks;         // 16-byte chunks per (token, head) row
    const int half = a.n_kv_heads * cpr;  // chunks of K (then as many of V) per token
    const int per_token = 2 * half;
    const int total = (t1 - t0) * per_token;
    const char* kb = static_cast<const char*>(a.k);
    const char* vb = static_cast<const char*>(a.v);
    char* kp = static_cast<char*>(a.k_pool);
    char* vp = static_cast<char*>(a.v_pool);

    int p0 = 0, colA = 0, stop = 0;
    for (int base = 0; base < total; base += 256 * kWriteBatch) {
        // 1. source rows
        u32x4 val[kWriteBatch];
#pragma unroll
        for (int j = 0; j < kWriteBatch; ++j) {
            const int c = base + j * 256 + (int)threadIdx.x;
            if (c < total) {
                const int ti = c / per_token;
                const int cc = c - ti * per_token;
                const bool is_v = cc >= half;
                const int hc = is_v ? cc - half : cc;
                const int h = hc / cpr;
                const int t = t0 + ti;
                const int64_t src_el = is_v ? (int64_t)t * a.v_stride_token + (int64_t)h * a.v_stride_head
                                            : (int64_t)t * a.k_stride_token + (int64_t)h * a.k_stride_head;
                val[j] = ld16((is_v ? vb : kb) + src_el * a.elem_bytes + (hc - h * cpr) * 16);
            }
        }
        // 2. destination pages (once): the first table column in [col0, colB]
        //    that cannot be written (-1, a block outside the pool, or past
        //    the table width) and the block ids of columns colA and colB.
        if (base == 0) {
            p0 = a.positions[q_begin];
            const int col0 = p0 / kPage;
            colA = (p0 + (t0 - q_begin)) / kPage;
            const int colB = (p0 + (t1 - 1 - q_begin)) / kPage;  // colA or colA + 1
            const int32_t* table = a.tables + (int64_t)b * a.table_stride;
            __syncthreads();  // the previous round's readers of s_stop / s_blk are done
            if (threadIdx.x == 0) s_stop = p0 < 0 ? -1 : 0x7fffffff;
            __syncthreads();
            if (p0 >= 0) {
                for (int c = col0 + (int)threadIdx.x; c <= colB; c += 256) {
                    const int blk = c < a.num_pages_per_seq ? table[c] : -1;
                    if (blk < 0 || (int64_t)blk >= a.num_blocks) atomicMin(&s_stop, c);
                    if (c == colA) s_blk[0] = blk;
                    if (c == colB) s_blk[1] = blk;
                }
            }
            __syncthreads();
            stop = s_stop;
        }
        // 3. stores (a token is written only if every column from col0 up to
        //    its own is valid)
#pragma unroll
        for (int j = 0; j < kWriteBatch; ++j) {
            const int c = base + j * 256 + (int)threadIdx.x;
            if (c < total) {
                const int ti = c / per_token;
                const int cc = c - ti * per_token;
                const int p = p0 + (t0 - q_begin) + ti;
                const int col = p / kPage;
                if (col < stop) {
                    const bool is_v = cc >= half;
                    const int hc = is_v ? cc - half : cc;
                    const int h = hc / cpr;
                    const int blk = s_blk[col == colA ? 0 : 1];
                    const int64_t dst_el = (int64_t)blk * a.pool_stride_block + (int64_t)h * a.pool_stride_head +
                                           (int64_t)(p % kPage) * a.pool_stride_row;
                    st16((is_v ? vp : kp) + dst_el * a.elem_bytes + (hc - h * cpr) * 16, val[j]);
                }
            }
        }
    }
    }
}

hipError_t launch_kv_cache_write(const CacheWriteArgs& a, int max_q_len, hipStream_t st) {
    if (a.num_seqs <= 0 || max_q_len <= 0) return hipSuccess;
    const dim3 grid((max_q_len + kWriteTokens - 1) / kWriteTokens, a.num_seqs);
    hipLaunchKernelGGL(kv_cache_write_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace femto
