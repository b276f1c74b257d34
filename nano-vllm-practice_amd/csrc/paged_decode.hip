// Paged decode attention (one query token per sequence) for gfx950.
//
// Semantics follow PagedAttentionGemvKernel
// (csrc/paged_attention/paged_attention_gemv.cu:16-221 of the reference):
// out[h, b] = softmax(q[h, b] . K_b^T / sqrt(D)) . V_b over kv_lens[b] keys,
// key j of sequence b at k_pool[tables[b][j / 16], h / n_rep, j % 16].
//
// Design (memory-bound GEMV):
//  * one workgroup = (split of the sequence's pages, KV head, head group of
//    NREP query heads); every K/V byte is loaded once and used by all NREP
//    query heads that share the KV head (the reference loads it n_rep times);
//  * 4 waves take the split's pages round-robin; inside a wave, DPP row r
//    (16 lanes) owns page rows r, r+4, r+8, r+12 and lane c of the row owns 8
//    head dims, so each K/V page is 4 coalesced 16-byte loads per lane
//    (bf16/f16; f32 uses 8) and the q.k reduction stays inside a DPP row;
//  * block ids are fetched 64 at a time (one per lane) and broadcast with
//    readlane, and each wave keeps two pages of loads in flight, so the
//    table never adds a dependent load per page;
//  * every lane keeps an online-softmax state (max, sum, 8 accumulators) per
//    query head over the keys it saw; states merge across DPP rows with
//    shuffles and across waves through LDS; split sequences leave one
//    partial state per split in the workspace and a small merge kernel on
//    the same stream combines them (no cross-workgroup fences or atomics,
//    which on gfx950 would write back and invalidate the XCD's L2);
//  * rows past kv_len are never read (loads are clamped to the last visible
//    row and their scores masked) and block ids outside the pool are never
//    dereferenced (their page reads as zeros), so NaN in unused pool memory
//    cannot leak.
#include "common.h"
#include "launch.h"

namespace femto {

// 8 values of a head-dim row owned by lane chunk c (0..15).
template <typename E>
struct RowSlice;

template <>
struct RowSlice<BF16> {
    u32x4 w;
    __device__ __forceinline__ void load(const char* row, int c) { w = ld16(row + 16 * c); }
    __device__ __forceinline__ void zero() { w = u32x4{0, 0, 0, 0}; }
    __device__ __forceinline__ void to_float(float f[8]) const { unpack8(BF16{}, w, f); }
    static __device__ __forceinline__ int dim(int c, int e) { return 8 * c + e; }
};

template <>
struct RowSlice<F16> {
    u32x4 w;
    __device__ __forceinline__ void load(const char* row, int c) { w = ld16(row + 16 * c); }
    __device__ __forceinline__ void zero() { w = u32x4{0, 0, 0, 0}; }
    __device__ __forceinline__ void to_float(float f[8]) const { unpack8(F16{}, w, f); }
    static __device__ __forceinline__ int dim(int c, int e) { return 8 * c + e; }
};

// f32: dims [4c, 4c+4) and [64+4c, 64+4c+4) so that each 16-byte load
// instruction of a DPP row covers 256 contiguous bytes.
template <>
struct RowSlice<F32> {
    u32x4 a, b;
    __device__ __forceinline__ void load(const char* row, int c) {
        a = ld16(row + 16 * c);
        b = ld16(row + 256 + 16 * c);
    }
    __device__ __forceinline__ void zero() {
        a = u32x4{0, 0, 0, 0};
        b = u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ void to_float(float f[8]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = __uint_as_float(a[i]);
            f[4 + i] = __uint_as_float(b[i]);
        }
    }
    static __device__ __forceinline__ int dim(int c, int e) { return e < 4 ? 4 * c + e : 64 + 4 * c + (e - 4); }
};

template <typename E>
__device__ __forceinline__ void store_elem(char* base, int64_t idx, float v);
template <>
__device__ __forceinline__ void store_elem<BF16>(char* base, int64_t idx, float v) {
    reinterpret_cast<__bf16*>(base)[idx] = (__bf16)v;
}
template <>
__device__ __forceinline__ void store_elem<F16>(char* base, int64_t idx, float v) {
    reinterpret_cast<_Float16*>(base)[idx] = (_Float16)v;
}
template <>
__device__ __forceinline__ void store_elem<F32>(char* base, int64_t idx, float v) {
    reinterpret_cast<float*>(base)[idx] = v;
}

// Running max sentinel: finite, so exp2(m_old - m_new) stays well defined
// while a lane has seen no visible key.
constexpr float kEmptyMax = -1.0e30f;

// K and V rows of one page held by a lane: page rows rg, rg+4, rg+8, rg+12.
template <typename E>
struct PageRegs {
    RowSlice<E> k[4], v[4];
};

template <typename E, int NREP>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
    constexpr int EB = E::kBytes;
    const int s = blockIdx.x;
    const int kvhg = blockIdx.y;
    const int b = blockIdx.z;
    const int kvh = kvhg / a.head_groups;
    const int hg = kvhg - kvh * a.head_groups;
    const int h0 = kvh * a.n_rep + hg * NREP;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rg = lane >> 4;
    const int c = lane & 15;

    const int kv_len = a.kv_lens[b];
    const int npages = kv_len > 0 ? (kv_len + kPage - 1) / kPage : 0;
    int nsplit = (npages + a.split_pages - 1) / a.split_pages;
    nsplit = nsplit < (int)gridDim.x ? nsplit : (int)gridDim.x;

    char* out = reinterpret_cast<char*>(a.out);
    if (kv_len <= 0) {
        // Empty context: the reference's P.V loop never runs and its zero
        // accumulator is stored (paged_attention_gemv.cu:203-218).
        if (s == 0) {
            for (int idx = tid; idx < NREP * kDimHead; idx += 256) {
                const int r = idx / kDimHead, d = idx - r * kDimHead;
                store_elem<E>(out, (int64_t)(h0 + r) * a.out_stride_head + (int64_t)b * a.out_stride_seq + d, 0.0f);
            }
        }
        return;
    }
    if (s >= nsplit) return;
    const int p0 = s * a.split_pages;
    const int p1 = (s == nsplit - 1) ? npages : p0 + a.split_pages;

    // Query rows of the NREP heads, in this lane's 8 dims.
    float qf[NREP][8];
    const char* qbase = reinterpret_cast<const char*>(a.q);
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        RowSlice<E> qs;
        qs.load(qbase + ((int64_t)(h0 + r) * a.q_stride_head + (int64_t)b * a.q_stride_seq) * EB, c);
        qs.to_float(qf[r]);
    }

    float m[NREP], l[NREP], acc[NREP][8];
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        m[r] = kEmptyMax;
        l[r] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
    }

    // This wave owns pages p0 + wave + 4*i, i < n_mine.  Their block ids are
    // fetched 64 at a time, one per lane, and broadcast with readlane.
    const int n_mine = (p1 - p0 - wave + 3) >> 2;
    const int32_t* table = a.tables + (int64_t)b * a.table_stride;
    const char* kpool = reinterpret_cast<const char*>(a.k_pool);
    const char* vpool = reinterpret_cast<const char*>(a.v_pool);
    const int64_t head_off = (int64_t)kvh * a.pool_stride_head;
    int tbl = -1;

    auto fetch_table = [&](int i0) {
        const int pg = p0 + wave + 4 * (i0 + lane);
        tbl = (i0 + lane < n_mine && pg < a.num_pages_per_seq) ? table[pg] : -1;
    };
    // Issue the 8 (f32: 16) 16-byte loads of page i.  Rows past kv_len are
    // clamped to the last visible row and blocks outside the pool to block 0,
    // so every load is in bounds and unconditional; those values are never
    // used (masked scores, zeroed registers).
    auto issue = [&](int i, PageRegs<E>& pr, bool& blk_ok) {
        const int blk = __builtin_amdgcn_readlane(tbl, i & 63);
        blk_ok = blk >= 0 && (int64_t)blk < a.num_blocks;
        const int pg = p0 + wave + 4 * i;
        const int last_row = kv_len - 1 - pg * kPage;
        const int64_t page_off = ((int64_t)(blk_ok ? blk : 0) * a.pool_stride_block + head_off) * EB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = min(rg + 4 * j, last_row);
            const int64_t off = page_off + (int64_t)row * a.pool_stride_row * EB;
            pr.k[j].load(kpool + off, c);
            pr.v[j].load(vpool + off, c);
        }
    };
    auto consume = [&](int i, PageRegs<E>& pr, bool blk_ok) {
        if (!blk_ok) {
            // A block id outside the pool reads as a page of zeros.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pr.k[j].zero();
                pr.v[j].zero();
            }
        }
        const int pg = p0 + wave + 4 * i;
        float sc[NREP][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float kf[8];
            pr.k[j].to_float(kf);
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qf[r][e], kf[e], d);
                sc[r][j] = d;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool valid = (pg * kPage + rg + 4 * j) < kv_len;
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const float t = row16_sum(sc[r][j]) * a.scale_log2;
                sc[r][j] = valid ? t : -INFINITY;
            }
        }
        float vf[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j) pr.v[j].to_float(vf[j]);
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            const float mx = fmaxf(fmaxf(sc[r][0], sc[r][1]), fmaxf(sc[r][2], sc[r][3]));
            const float mn = fmaxf(m[r], mx);
            const float al = fast_exp2(m[r] - mn);
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = fast_exp2(sc[r][j] - mn);
            l[r] = fmaf(l[r], al, (p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float t = acc[r][e] * al;
                t = fmaf(p[0], vf[0][e], t);
                t = fmaf(p[1], vf[1][e], t);
                t = fmaf(p[2], vf[2][e], t);
                t = fmaf(p[3], vf[3][e], t);
                acc[r][e] = t;
            }
            m[r] = mn;
        }
    };

    // Two pages in flight per wave: page i+1 loads while page i computes.
    PageRegs<E> ra, rb;
    bool ok_a = false, ok_b = false;
    if (n_mine > 0) {
        fetch_table(0);
        issue(0, ra, ok_a);
    }
    for (int i = 0; i < n_mine; i += 2) {
        if (i + 1 < n_mine) {
            if (((i + 1) & 63) == 0) fetch_table(i + 1);
            issue(i + 1, rb, ok_b);
        }
        consume(i, ra, ok_a);
        if (i + 1 < n_mine) {
            if (i + 2 < n_mine) {
                if (((i + 2) & 63) == 0) fetch_table(i + 2);
                issue(i + 2, ra, ok_a);
            }
            consume(i + 1, rb, ok_b);
        }
    }

    // Merge the four DPP rows of the wave (they hold the same dims).
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
#pragma unroll
        for (int sh = 16; sh <= 32; sh *= 2) {
            const float mo = shfl_xor_f32(m[r], sh);
            const float lo = shfl_xor_f32(l[r], sh);
            const float mn = fmaxf(m[r], mo);
            const float fa = fast_exp2(m[r] - mn);
            const float fb = fast_exp2(mo - mn);
            l[r] = l[r] * fa + lo * fb;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float ao = shfl_xor_f32(acc[r][e], sh);
                acc[r][e] = acc[r][e] * fa + ao * fb;
            }
            m[r] = mn;
        }
    }

    __shared__ float s_acc[4][NREP][kDimHead];
    __shared__ float s_ml[4][NREP][2];
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

    const int H = a.n_heads;
    const int S = a.max_splits;
    for (int idx = tid; idx < NREP * kDimHead; idx += 256) {
        const int r = idx / kDimHead, d = idx - r * kDimHead;
        float M = s_ml[0][r][0];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, s_ml[w][r][0]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = fast_exp2(s_ml[w][r][0] - M);
            L = fmaf(s_ml[w][r][1], f, L);
            O = fmaf(s_acc[w][r][d], f, O);
        }
        const int h = h0 + r;
        if (nsplit == 1) {
            store_elem<E>(out, (int64_t)h * a.out_stride_head + (int64_t)b * a.out_stride_seq + d, O / L);
        } else {
            // Partial state of this split; paged_decode_merge_kernel combines them.
            const int64_t slot = ((int64_t)b * H + h) * S + s;
            a.part_acc[slot * kDimHead + d] = O;
            if (d == 0) {
                a.part_ml[slot * 2] = M;
                a.part_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// Combine the split partials of sequences that were split; one workgroup per
// (sequence, query head), one thread per head dim.  Runs after the split
// kernel on the same stream, so no cross-workgroup synchronisation is needed.
template <typename E>
__global__ __launch_bounds__(128) void paged_decode_merge_kernel(DecodeArgs a) {
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int d = threadIdx.x;
    const int kv_len = a.kv_lens[b];
    const int npages = kv_len > 0 ? (kv_len + kPage - 1) / kPage : 0;
    int nsplit = (npages + a.split_pages - 1) / a.split_pages;
    nsplit = nsplit < a.max_splits ? nsplit : a.max_splits;
    if (nsplit <= 1) return;
    const int64_t slot0 = ((int64_t)b * a.n_heads + h) * a.max_splits;
    float M = kEmptyMax;
    for (int i = 0; i < nsplit; ++i) M = fmaxf(M, a.part_ml[(slot0 + i) * 2]);
    float L = 0.0f, O = 0.0f;
    for (int i = 0; i < nsplit; ++i) {
        const float f = fast_exp2(a.part_ml[(slot0 + i) * 2] - M);
        L = fmaf(a.part_ml[(slot0 + i) * 2 + 1], f, L);
        O = fmaf(a.part_acc[(slot0 + i) * kDimHead + d], f, O);
    }
    store_elem<E>(reinterpret_cast<char*>(a.out), (int64_t)h * a.out_stride_head + (int64_t)b * a.out_stride_seq + d,
                  O / L);
}

template <typename E, int NREP>
static hipError_t launch_t(const DecodeArgs& a, int grid_splits, int grid_heads, int num_seqs, hipStream_t st) {
    dim3 grid(grid_splits, grid_heads, num_seqs);
    hipLaunchKernelGGL((paged_decode_kernel<E, NREP>), grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || grid_splits <= 1) return e;
    hipLaunchKernelGGL((paged_decode_merge_kernel<E>), dim3(a.n_heads, num_seqs), dim3(kDimHead), 0, st, a);
    return hipGetLastError();
}

template <typename E>
static hipError_t launch_e(const DecodeArgs& a, int nrep_tile, int grid_splits, int grid_heads, int num_seqs,
                           hipStream_t st) {
    switch (nrep_tile) {
        case 1: return launch_t<E, 1>(a, grid_splits, grid_heads, num_seqs, st);
        case 2: return launch_t<E, 2>(a, grid_splits, grid_heads, num_seqs, st);
        case 4: return launch_t<E, 4>(a, grid_splits, grid_heads, num_seqs, st);
        case 8: return launch_t<E, 8>(a, grid_splits, grid_heads, num_seqs, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_paged_decode(int dtype, const DecodeArgs& a, int nrep_tile, int grid_splits, int num_seqs,
                               hipStream_t st) {
    const int grid_heads = a.n_heads / nrep_tile;
    if (grid_splits <= 0 || num_seqs <= 0 || grid_heads <= 0) return hipSuccess;
    switch (dtype) {
        case kDtypeF32: return launch_e<F32>(a, nrep_tile, grid_splits, grid_heads, num_seqs, st);
        case kDtypeF16: return launch_e<F16>(a, nrep_tile, grid_splits, grid_heads, num_seqs, st);
        case kDtypeBF16: return launch_e<BF16>(a, nrep_tile, grid_splits, grid_heads, num_seqs, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace femto
