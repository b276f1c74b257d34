// Device-side build of the varlen attention metadata.
//
// Rules of the reference's ModelRunner (femtovllm/engine/model_runner.py):
// for scheduled sequence b with pos = num_computed[b] and n = num_tokens[b],
// kv_len = pos + n, positions = pos .. kv_len - 1, cu_seqlens is the prefix
// sum of n, each sequence has ceil(n / Q_TILE_SIZE) query tiles (cu_q_tiles
// and q_tile_to_seq_idx), lines 187-202; a decode step is the case n = 1
// (283-293); block tables are padded with -1 to the longest (46-72).  The
// host gives the per-sequence counts and the block tables in CSR form
// (offsets + flat ids) in one buffer; two kernels fill every tensor.
#include "common.h"
#include "launch.h"

namespace femto {

// One workgroup: prefix sums over the sequences, 256 at a time.
__global__ __launch_bounds__(256) void metadata_scan_kernel(MetadataArgs a) {
    __shared__ int s_tok[4], s_til[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int carry_tok = 0, carry_til = 0;
    if (tid == 0) {
        a.cu_seqlens[0] = 0;
        a.cu_q_tiles[0] = 0;
    }
    for (int base = 0; base < a.num_seqs; base += 256) {
        const int i = base + tid;
        const int n = i < a.num_seqs ? a.num_tokens[i] : 0;
        const int til = (n + a.q_tile_size - 1) / a.q_tile_size;
        int st = n, sq = til;  // inclusive scans within the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int ut = __shfl_up(st, o, 64), uq = __shfl_up(sq, o, 64);
            if (lane >= o) {
                st += ut;
                sq += uq;
            }
        }
        if (lane == 63) {
            s_tok[wave] = st;
            s_til[wave] = sq;
        }
        __syncthreads();
        int off_t = carry_tok, off_q = carry_til, tot_t = 0, tot_q = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            off_t += w < wave ? s_tok[w] : 0;
            off_q += w < wave ? s_til[w] : 0;
            tot_t += s_tok[w];
            tot_q += s_til[w];
        }
        __syncthreads();
        if (i < a.num_seqs) {
            a.cu_seqlens[i + 1] = off_t + st;
            a.cu_q_tiles[i + 1] = off_q + sq;
            a.kv_lens[i] = a.num_computed[i] + n;
        }
        carry_tok += tot_t;
        carry_til += tot_q;
    }
}

// Workgroup (x, b): entries 256x .. 256x + 255 of sequence b's positions,
// query-tile map and block-table row.
__global__ __launch_bounds__(256) void metadata_fill_kernel(MetadataArgs a) {
    const int b = blockIdx.y;
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    const int n = a.num_tokens[b];
    if (i < n) a.positions[a.cu_seqlens[b] + i] = a.num_computed[b] + i;
    const int til = (n + a.q_tile_size - 1) / a.q_tile_size;
    if (i < til) a.q_tile_to_seq_idx[a.cu_q_tiles[b] + i] = b;
    if (i < a.table_width) {
        const int off = a.block_offsets[b];
        const int cnt = a.block_offsets[b + 1] - off;
        a.block_tables[(int64_t)b * a.table_width + i] = i < cnt ? a.block_ids[off + i] : -1;
    }
}

hipError_t launch_varlen_metadata(const MetadataArgs& a, int max_q_len, hipStream_t st) {
    if (a.num_seqs <= 0) return hipSuccess;
    hipLaunchKernelGGL(metadata_scan_kernel, dim3(1), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int span = max(max(max_q_len, a.table_width), 1);  // tiles <= tokens
    hipLaunchKernelGGL(metadata_fill_kernel, dim3((span + 255) / 256, a.num_seqs), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace femto
