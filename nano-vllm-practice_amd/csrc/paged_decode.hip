// Paged decode attention (one query token per sequence) for gfx950.
//
// Semantics follow PagedAttentionGemvKernel
// (csrc/paged_attention/paged_attention_gemv.cu:16-221 of the reference):
// out[h, b] = softmax(q[h, b] . K_b^T / sqrt(D)) . V_b over kv_lens[b] keys,
// key j of sequence b at k_pool[tables[b][j / 16], h / n_rep, j % 16].
//
// Design (memory-bound GEMV):
//  * waves are independent workers: per group of NREP query heads sharing a
//    KV head, the pages of all sequences are concatenated and cut into equal
//    slices, one per wave (one wave per SIMD); every K/V byte is loaded once
//    and used by all NREP query heads (the reference loads it n_rep times);
//  * inside a wave, DPP row r (16 lanes) owns page rows r, r+4, r+8, r+12 and
//    lane c of the row owns 8 head dims, so each K/V page is 4 coalesced
//    16-byte loads per lane (bf16/f16; f32 uses 8), issued with the
//    non-temporal hint (each byte is read once per call), and the q.k
//    reduction stays inside a DPP row;
//  * block ids are fetched 64 at a time (one per lane) and broadcast with
//    readlane, and each wave keeps three pages of loads in flight, so the
//    table never adds a dependent load per page;
//  * every lane keeps an online-softmax state (max, sum, 8 accumulators) per
//    query head over the keys it saw; states merge across the four DPP rows
//    with permlane swaps, each sequence segment of a slice leaves one partial
//    state in the workspace, and a small merge kernel on the same stream
//    combines them (no cross-workgroup fences or atomics, which on gfx950
//    would write back and invalidate the XCD's L2);
//  * rows past kv_len are never read (loads are clamped to the last visible
//    row and their scores masked) and block ids outside the pool are never
//    dereferenced (their page reads as zeros), so NaN in unused pool memory
//    cannot leak.
#include "decode_worker.h"

namespace femto {

template <typename E, int NREP, bool FULL>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
    decode_waves<E, NREP, FULL>(a, blockIdx.x);
}

// One-launch decode for calls of short contexts: one workgroup of W waves per
// (sequence, KV head group), wave w taking the w-th of W contiguous shares
// of the sequence's pages; the waves fold their states through LDS and
// write the normalised rows, so no workspace and no merge launch are needed.
// Decode calls only (query row b, kv_lens[b] keys).  W = 4; calls with few
// (sequence, query head) pairs run one query head per wave with W = 8, so
// each wave walks half as many pages (a wave's page math, not the loads,
// sets the length of such a call).
template <typename E, int NREP, bool FULL, int W>
__global__ __launch_bounds__(64 * W) void paged_decode_single_kernel(DecodeArgs a) {
    __shared__ float s_ml[W][NREP][2];
    __shared__ float s_acc[W][NREP][kDimHead];
    const int b = blockIdx.x, grp = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, rg = lane >> 4;
    const int kvh = grp / a.head_groups;
    const int h0 = kvh * a.n_rep + (grp - kvh * a.head_groups) * NREP;
    const int kv_len = a.kv_lens[b];
    const int npg = pages_of(kv_len);
    const int per = (npg + W - 1) / W;
    const int lp0 = min(npg, wave * per), lp1 = min(npg, lp0 + per);
    float m[NREP], l[NREP], acc[NREP][8];
    if (lp1 > lp0) {
        decode_segment<E, NREP, FULL>(a, b, kv_len, lp0, lp1 - lp0, b, h0, (int64_t)kvh * a.pool_stride_head, m, l,
                                      acc);
    } else {
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            m[r] = kEmptyMax;
            l[r] = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
        }
    }
    if (rg == 0) {
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s_acc[wave][r][RowSlice<E>::dim(c, e)] = acc[r][e];
            if (c == 0) {
                s_ml[wave][r][0] = m[r];
                s_ml[wave][r][1] = l[r];
            }
        }
    }
    __syncthreads();
    char* out = reinterpret_cast<char*>(a.out);
    for (int i = threadIdx.x; i < NREP * kDimHead; i += 64 * W) {
        const int r = i / kDimHead, d = i - r * kDimHead;
        if (!FULL && d >= a.head_dim) continue;
        const int64_t o = (int64_t)(h0 + r) * a.out_stride_head + (int64_t)b * a.out_stride_seq + d;
        if (npg == 0) {  // empty context: the reference stores its zero accumulator
            store_elem<E>(out, o, 0.0f);
            continue;
        }
        float M = kEmptyMax;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, s_ml[w][r][0]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float f = fast_exp2(s_ml[w][r][0] - M);
            L = fmaf(s_ml[w][r][1], f, L);
            O = fmaf(s_acc[w][r][d], f, O);
        }
        store_elem<E>(out, o, O / L);
    }
}

// Final softmax merge: one workgroup per (sequence, query head), one thread
// per head dim.  Runs after the split kernel on the same stream.
template <typename E>
__global__ __launch_bounds__(128) void paged_decode_merge_kernel(DecodeArgs a) {
    __shared__ float s_w[128];  // slot maxima
    __shared__ float s_lv[128];  // slot sums
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int t = threadIdx.x;
    char* out = reinterpret_cast<char*>(a.out);
    int row, kvl;
    if (!decode_row_of(a, b, row, kvl)) return;  // a prefill row (whole workgroup)
    const int64_t o = (int64_t)h * a.out_stride_head + (int64_t)row * a.out_stride_seq + t;
    const int64_t sl0 = ((int64_t)b * a.n_heads + h) * a.max_slots;
    const float* src = a.part_acc + sl0 * kDimHead + t;
    // Every load that does not depend on another is issued first: kv_len,
    // the slot count, (m, l) of every slot this (sequence, head) may own and
    // the accumulators of its first kSpec slots (a sequence usually spans a
    // few slices).  Entries past the count are stale and are masked below.
    constexpr int kSpec = 4;
    const int count_ld = a.seq_slots[b];
    const float m_ld = t < a.max_slots ? a.part_ml[(sl0 + t) * 2] : kEmptyMax;
    const float l_ld = t < a.max_slots ? a.part_ml[(sl0 + t) * 2 + 1] : 0.0f;
    float v[kSpec];
#pragma unroll
    for (int i = 0; i < kSpec; ++i) v[i] = i < a.max_slots ? src[(int64_t)i * kDimHead] : 0.0f;
    if (kvl <= 0) {
        // Empty context.  Decode call: the reference's P.V loop never runs
        // and its zero accumulator is stored (paged_attention_gemv.cu:203-218).
        // Decode row of a prefill call: 0 / 0, NaN, as the prefill kernels
        // give for a row with no visible key.
        if (t < a.head_dim) store_elem<E>(out, o, a.cu_seqlens ? __builtin_nanf("") : 0.0f);
        return;
    }
    const int count = count_ld;
    // Thread i < count publishes slot i's (m, l); after one barrier every
    // thread folds the count slots itself (a sequence spans a few slices,
    // at most max_slots <= 128), so no further reduction round is needed.
    if (t < count) {
        s_w[t] = m_ld;
        s_lv[t] = l_ld;
    }
    __syncthreads();
    float M = kEmptyMax;
    for (int i = 0; i < count; ++i) M = fmaxf(M, s_w[i]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int i = 0; i < kSpec; ++i) {
        const float wi = i < count ? fast_exp2(s_w[i < count ? i : 0] - M) : 0.0f;
        L = fmaf(i < count ? s_lv[i] : 0.0f, wi, L);
        O = fmaf(i < count ? v[i] : 0.0f, wi, O);
    }
    for (int i = kSpec; i < count; ++i) {
        const float wi = fast_exp2(s_w[i] - M);
        L = fmaf(s_lv[i], wi, L);
        O = fmaf(src[(int64_t)i * kDimHead], wi, O);
    }
    if (t < a.head_dim) store_elem<E>(out, o, O / L);
}

// One wave per SIMD (4 per CU), each with three pages of K and V in flight
// (96 KB per CU).  HBM read throughput peaks there: more resident waves queue
// more requests and lose bandwidth (on the 545 MB Qwen3-0.6B-shaped batch, 16
// waves per CU ran at 4.85 TB/s and 4 per CU at 5.2 TB/s with ordinary loads;
// 8 per CU with non-temporal loads was 2 % slower than 4, and 6 or 8 per CU
// 3-12 % slower with the dot2 page math).  Sets a.waves_per_group and returns
// the workgroups of 4 waves that cover the workers (0 on a device error).
int decode_worker_blocks(DecodeArgs& a) {
    int cus = 0;
    if (device_cu_count(cus) != hipSuccess) return 0;
    const int total_waves = cus * 4;
    a.waves_per_group = total_waves / a.grid_heads > 0 ? total_waves / a.grid_heads : 1;
    return (a.waves_per_group * a.grid_heads + 3) / 4;
}

template <typename E>
static hipError_t launch_merge_t(const DecodeArgs& a, int num_seqs, hipStream_t st) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<E>), dim3(a.n_heads, num_seqs), dim3(kDimHead), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_paged_decode_merge(int dtype, const DecodeArgs& a, int num_seqs, hipStream_t st) {
    switch (dtype) {
        case kDtypeF32: return launch_merge_t<F32>(a, num_seqs, st);
        case kDtypeF16: return launch_merge_t<F16>(a, num_seqs, st);
        case kDtypeBF16: return launch_merge_t<BF16>(a, num_seqs, st);
        default: return hipErrorInvalidValue;
    }
}

template <typename E, int NREP, bool FULL>
static hipError_t launch_t(DecodeArgs a, int num_seqs, bool single, hipStream_t st) {
    if (single) {
        if constexpr (NREP == 1) {
            if (a.single_waves == 8) {
                hipLaunchKernelGGL((paged_decode_single_kernel<E, 1, FULL, 8>), dim3(num_seqs, a.grid_heads),
                                   dim3(512), 0, st, a);
                return hipGetLastError();
            }
        }
        hipLaunchKernelGGL((paged_decode_single_kernel<E, NREP, FULL, 4>), dim3(num_seqs, a.grid_heads), dim3(256), 0,
                           st, a);
        return hipGetLastError();
    }
    const int grid = decode_worker_blocks(a);
    if (grid <= 0) return hipErrorInvalidDevice;
    hipLaunchKernelGGL((paged_decode_kernel<E, NREP, FULL>), dim3(grid), dim3(256), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge_t<E>(a, num_seqs, st);
}

template <typename E, bool FULL>
static hipError_t launch_e(const DecodeArgs& a, int nrep_tile, int num_seqs, bool single, hipStream_t st) {
    switch (nrep_tile) {
        case 1: return launch_t<E, 1, FULL>(a, num_seqs, single, st);
        case 2: return launch_t<E, 2, FULL>(a, num_seqs, single, st);
        case 4: return launch_t<E, 4, FULL>(a, num_seqs, single, st);
        case 8:
            if constexpr (!std::is_same<E, F32>::value) return launch_t<E, 8, FULL>(a, num_seqs, single, st);
            return hipErrorInvalidValue;  // f32 plans stop at 4 heads per wave
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_paged_decode(int dtype, const DecodeArgs& a, int nrep_tile, int num_seqs, bool single,
                               hipStream_t st) {
    if (num_seqs <= 0 || a.grid_heads <= 0) return hipSuccess;
    if (single && a.cu_seqlens) return hipErrorInvalidValue;  // decode calls only
    if (a.head_dim <= 0 || a.head_dim > kDimHead) return hipErrorInvalidValue;
    const bool full = a.head_dim == kDimHead;
    switch (dtype) {
        case kDtypeF32: return full ? launch_e<F32, true>(a, nrep_tile, num_seqs, single, st)
                                    : launch_e<F32, false>(a, nrep_tile, num_seqs, single, st);
        case kDtypeF16: return full ? launch_e<F16, true>(a, nrep_tile, num_seqs, single, st)
                                    : launch_e<F16, false>(a, nrep_tile, num_seqs, single, st);
        case kDtypeBF16: return full ? launch_e<BF16, true>(a, nrep_tile, num_seqs, single, st)
                                     : launch_e<BF16, false>(a, nrep_tile, num_seqs, single, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace femto
