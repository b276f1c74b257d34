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
    __device__ __forceinline__ void stream(const char* row, int c) { w = ld16_nt(row + 16 * c); }
    __device__ __forceinline__ void zero() { w = u32x4{0, 0, 0, 0}; }
    __device__ __forceinline__ void to_float(float f[8]) const { unpack8(BF16{}, w, f); }
    static __device__ __forceinline__ int dim(int c, int e) { return 8 * c + e; }
};

template <>
struct RowSlice<F16> {
    u32x4 w;
    __device__ __forceinline__ void load(const char* row, int c) { w = ld16(row + 16 * c); }
    __device__ __forceinline__ void stream(const char* row, int c) { w = ld16_nt(row + 16 * c); }
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
    __device__ __forceinline__ void stream(const char* row, int c) {
        a = ld16_nt(row + 16 * c);
        b = ld16_nt(row + 256 + 16 * c);
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

__device__ __forceinline__ int pages_of(int kv_len) { return kv_len > 0 ? (kv_len + kPage - 1) / kPage : 0; }

// Load-balanced split-KV decode.  Every wave is an independent worker: the
// pages of all sequences are concatenated (per KV head group) and cut into
// equal slices of C pages, one slice per wave, with as many waves as the GPU
// holds at once.  A wave walks its slice sequence by sequence and leaves one
// partial softmax state per (sequence segment, query head); the merge kernel
// combines them.  Slice s of sequence b is partial slot s - first_wave(b).
template <typename E, int NREP>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeArgs a) {
    constexpr int EB = E::kBytes;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int grp = gw / a.waves_per_group;
    const int wi = gw - grp * a.waves_per_group;
    if (grp >= a.grid_heads) return;  // waves are independent: no barriers below
    const int kvh = grp / a.head_groups;
    const int hg = grp - kvh * a.head_groups;
    const int h0 = kvh * a.n_rep + hg * NREP;
    const int rg = lane >> 4;
    const int c = lane & 15;
    const int B = a.num_seqs;

    // Pass 1: total pages P and the longest sequence; slice length C.
    int total = 0, longest = 0;
#pragma unroll 4
    for (int i = lane; i < B; i += kWave) {
        const int pg = pages_of(a.kv_lens[i]);
        total += pg;
        longest = max(longest, pg);
    }
    total = wave_sum_i32(total);
    longest = wave_max_i32(longest);
    int C = (total + a.waves_per_group - 1) / a.waves_per_group;
    C = max(C, a.min_chunk_pages);
    C = max(C, (longest + a.max_slots - 2) / (a.max_slots - 1));  // at most max_slots slots per sequence
    C = max(C, 1);
    const int x0 = wi * C;
    if (x0 >= total) return;
    const int x1 = min(total, x0 + C);

    // Pass 2: the sequence holding page x0.  Lane i of the current 64-wide
    // chunk keeps kv_len and the exclusive page prefix of sequence base + i.
    int base = 0, carry = 0, my_len = 0, my_excl = 0, chunk_total = 0;
    for (;; base += kWave) {
        const int i = base + lane;
        my_len = i < B ? a.kv_lens[i] : 0;
        const int pg = pages_of(my_len);
        const int incl = wave_incl_scan_i32(pg);
        my_excl = carry + incl - pg;
        chunk_total = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (x0 < carry + chunk_total) break;
        carry += chunk_total;
    }
    // first sequence of the chunk whose pages end after x0 (skips empty ones)
    const uint64_t after = __ballot(base + lane < B && my_excl + pages_of(my_len) > x0);
    int b = base + __builtin_ctzll(after);

    // Query rows of the NREP heads, in this lane's 8 dims.
    float qf[NREP][8];
    const char* qbase = reinterpret_cast<const char*>(a.q);
    const char* kpool = reinterpret_cast<const char*>(a.k_pool);
    const char* vpool = reinterpret_cast<const char*>(a.v_pool);
    const int64_t head_off = (int64_t)kvh * a.pool_stride_head;
    const int H = a.n_heads;

    int x = x0;
    while (x < x1) {
        if (b - base >= kWave) {  // next chunk of sequences
            carry += chunk_total;
            base += kWave;
            const int i = base + lane;
            my_len = i < B ? a.kv_lens[i] : 0;
            const int pg = pages_of(my_len);
            const int incl = wave_incl_scan_i32(pg);
            my_excl = carry + incl - pg;
            chunk_total = __builtin_amdgcn_readlane(incl, kWave - 1);
        }
        const int kv_len = __builtin_amdgcn_readlane(my_len, b - base);  // b - base is wave-uniform
        const int S = __builtin_amdgcn_readlane(my_excl, b - base);
        const int npg = pages_of(kv_len);
        if (npg == 0 || S + npg <= x) {
            ++b;
            continue;
        }
        const int lp0 = x - S;                 // first page of the segment
        const int lp1 = min(x1, S + npg) - S;  // one past its last page
        const int n = lp1 - lp0;

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

        const int32_t* table = a.tables + (int64_t)b * a.table_stride;
        int tbl = -1;
        auto fetch_table = [&](int i0) {
            const int pg = lp0 + i0 + lane;
            tbl = (i0 + lane < n && pg < a.num_pages_per_seq) ? table[pg] : -1;
        };
        // The 8 (f32: 16) 16-byte loads of page lp0 + i.  Rows past kv_len
        // are clamped to the last visible row and blocks outside the pool to
        // block 0, so every load is in bounds and unconditional; those values
        // are never used (masked scores, zeroed registers).
        auto issue = [&](int i, PageRegs<E>& pr, bool& blk_ok) {
            const int blk = __builtin_amdgcn_readlane(tbl, i & 63);
            blk_ok = blk >= 0 && (int64_t)blk < a.num_blocks;
            const int pg = lp0 + i;
            const int last_row = kv_len - 1 - pg * kPage;
            const int64_t page_off = ((int64_t)(blk_ok ? blk : 0) * a.pool_stride_block + head_off) * EB;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = min(rg + 4 * j, last_row);
                const int64_t off = page_off + (int64_t)row * a.pool_stride_row * EB;
                pr.k[j].stream(kpool + off, c);
                pr.v[j].stream(vpool + off, c);
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
            const int pg = lp0 + i;
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

        // Three pages in flight: pages i+1 and i+2 load while page i
        // computes (96 KB of loads per CU at one wave per SIMD).
        PageRegs<E> r0, r1, r2;
        bool k0 = false, k1 = false, k2 = false;
        fetch_table(0);
        issue(0, r0, k0);
        if (1 < n) issue(1, r1, k1);
        for (int i = 0; i < n; i += 3) {
            if (i + 2 < n) {
                if (((i + 2) & 63) == 0) fetch_table(i + 2);
                issue(i + 2, r2, k2);
            }
            consume(i, r0, k0);
            if (i + 1 < n) {
                if (i + 3 < n) {
                    if (((i + 3) & 63) == 0) fetch_table(i + 3);
                    issue(i + 3, r0, k0);
                }
                consume(i + 1, r1, k1);
                if (i + 2 < n) {
                    if (i + 4 < n) {
                        if (((i + 4) & 63) == 0) fetch_table(i + 4);
                        issue(i + 4, r1, k1);
                    }
                    consume(i + 2, r2, k2);
                }
            }
        }

        // Merge the four DPP rows (same dims, different keys): rows 0+1 and
        // 2+3, then the two halves; every lane of a pair ends with the pair's
        // state (the first row's terms first, as row 0 computes them).
        auto merge_pair = [&](auto pair) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                float m0, m1, l0, l1;
                pair(m[r], m0, m1);
                pair(l[r], l0, l1);
                const float mn = fmaxf(m0, m1);
                const float f0 = fast_exp2(m0 - mn);
                const float f1 = fast_exp2(m1 - mn);
                l[r] = l0 * f0 + l1 * f1;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float a0, a1;
                    pair(acc[r][e], a0, a1);
                    acc[r][e] = a0 * f0 + a1 * f1;
                }
                m[r] = mn;
            }
        };
        merge_pair([](float x, float& a, float& b) { pair16(x, a, b); });
        merge_pair([](float x, float& a, float& b) { pair32(x, a, b); });

        // Partial state of this segment.
        const int slot = wi - S / C;
        if (rg == 0) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const int64_t sl = ((int64_t)b * H + h0 + r) * a.max_slots + slot;
                float* dst = a.part_acc + sl * kDimHead;
#pragma unroll
                for (int e = 0; e < 8; ++e) dst[RowSlice<E>::dim(c, e)] = acc[r][e];
                if (c == 0) {
                    a.part_ml[sl * 2] = m[r];
                    a.part_ml[sl * 2 + 1] = l[r];
                }
            }
        }
        if (lane == 0 && grp == 0 && lp1 == npg) a.seq_slots[b] = slot + 1;  // last segment: slot count
        x = S + lp1;
        ++b;
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
    const int64_t o = (int64_t)h * a.out_stride_head + (int64_t)b * a.out_stride_seq + t;
    const int64_t sl0 = ((int64_t)b * a.n_heads + h) * a.max_slots;
    const float* src = a.part_acc + sl0 * kDimHead + t;
    // Every load that does not depend on another is issued first: kv_len,
    // the slot count, (m, l) of every slot this (sequence, head) may own and
    // the accumulators of its first kSpec slots (a sequence usually spans a
    // few slices).  Entries past the count are stale and are masked below.
    constexpr int kSpec = 4;
    const int kvl = a.kv_lens[b];
    const int count_ld = a.seq_slots[b];
    const float m_ld = t < a.max_slots ? a.part_ml[(sl0 + t) * 2] : kEmptyMax;
    const float l_ld = t < a.max_slots ? a.part_ml[(sl0 + t) * 2 + 1] : 0.0f;
    float v[kSpec];
#pragma unroll
    for (int i = 0; i < kSpec; ++i) v[i] = i < a.max_slots ? src[(int64_t)i * kDimHead] : 0.0f;
    if (kvl <= 0) {
        // Empty context: the reference's P.V loop never runs and its zero
        // accumulator is stored (paged_attention_gemv.cu:203-218).
        store_elem<E>(out, o, 0.0f);
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
    store_elem<E>(out, o, O / L);
}

template <typename E, int NREP>
static hipError_t launch_t(DecodeArgs a, int num_seqs, hipStream_t st) {
    // One wave per SIMD (4 per CU), each with three pages of K and V in
    // flight (96 KB per CU).  HBM read throughput peaks there: more resident
    // waves queue more requests and lose bandwidth (on the 545 MB
    // Qwen3-0.6B-shaped batch, 16 waves per CU ran at 4.85 TB/s and 4 per CU
    // at 5.2 TB/s with ordinary loads; 8 per CU with non-temporal loads was
    // 2 % slower than 4).
    static int cu_count[64] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int& cus = cu_count[dev & 63];
    if (cus == 0) {
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        if (cus <= 0) cus = 1;
    }
    const int total_waves = cus * 4;
    a.waves_per_group = total_waves / a.grid_heads > 0 ? total_waves / a.grid_heads : 1;
    const int grid = (a.waves_per_group * a.grid_heads + 3) / 4;
    hipLaunchKernelGGL((paged_decode_kernel<E, NREP>), dim3(grid), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((paged_decode_merge_kernel<E>), dim3(a.n_heads, num_seqs), dim3(kDimHead), 0, st, a);
    return hipGetLastError();
}

template <typename E>
static hipError_t launch_e(const DecodeArgs& a, int nrep_tile, int num_seqs, hipStream_t st) {
    switch (nrep_tile) {
        case 1: return launch_t<E, 1>(a, num_seqs, st);
        case 2: return launch_t<E, 2>(a, num_seqs, st);
        case 4: return launch_t<E, 4>(a, num_seqs, st);
        case 8: return launch_t<E, 8>(a, num_seqs, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_paged_decode(int dtype, const DecodeArgs& a, int nrep_tile, int num_seqs, hipStream_t st) {
    if (num_seqs <= 0 || a.grid_heads <= 0) return hipSuccess;
    switch (dtype) {
        case kDtypeF32: return launch_e<F32>(a, nrep_tile, num_seqs, st);
        case kDtypeF16: return launch_e<F16>(a, nrep_tile, num_seqs, st);
        case kDtypeBF16: return launch_e<BF16>(a, nrep_tile, num_seqs, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace femto
