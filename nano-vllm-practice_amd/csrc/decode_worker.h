// Decode wave workers (one query token per sequence), shared by the decode
// kernel (paged_decode.hip) and the fused prefill launch that runs a mixed
// batch's decode rows beside its prefill tiles (paged_prefill.hip).
#pragma once

#include <type_traits>

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
    // head_dim D < 128: chunks at or past D are not read and hold zeros
    __device__ __forceinline__ void load_d(const char* row, int c, int D) {
        if (8 * c < D) load(row, c);
        else zero();
    }
    __device__ __forceinline__ void stream_d(const char* row, int c, int D) {
        if (8 * c < D) stream(row, c);
        else zero();
    }
    __device__ __forceinline__ void to_float(float f[8]) const { unpack8(BF16{}, w, f); }
    // sum over the 8 dims of this * o, products exact, fp32 accumulation
    __device__ __forceinline__ float dot(const RowSlice& o) const {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, (uint32_t)w[i]),
                                                __builtin_bit_cast(bf16x2, (uint32_t)o.w[i]), d, false);
        return d;
    }
    static __device__ __forceinline__ int dim(int c, int e) { return 8 * c + e; }
};

template <>
struct RowSlice<F16> {
    u32x4 w;
    __device__ __forceinline__ void load(const char* row, int c) { w = ld16(row + 16 * c); }
    __device__ __forceinline__ void stream(const char* row, int c) { w = ld16_nt(row + 16 * c); }
    __device__ __forceinline__ void zero() { w = u32x4{0, 0, 0, 0}; }
    __device__ __forceinline__ void load_d(const char* row, int c, int D) {
        if (8 * c < D) load(row, c);
        else zero();
    }
    __device__ __forceinline__ void stream_d(const char* row, int c, int D) {
        if (8 * c < D) stream(row, c);
        else zero();
    }
    __device__ __forceinline__ void to_float(float f[8]) const { unpack8(F16{}, w, f); }
    __device__ __forceinline__ float dot(const RowSlice& o) const {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, (uint32_t)w[i]),
                                       __builtin_bit_cast(f16x2, (uint32_t)o.w[i]), d, false);
        return d;
    }
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
    __device__ __forceinline__ void load_d(const char* row, int c, int D) {
        a = 4 * c < D ? ld16(row + 16 * c) : u32x4{0, 0, 0, 0};
        b = 64 + 4 * c < D ? ld16(row + 256 + 16 * c) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ void stream_d(const char* row, int c, int D) {
        a = 4 * c < D ? ld16_nt(row + 16 * c) : u32x4{0, 0, 0, 0};
        b = 64 + 4 * c < D ? ld16_nt(row + 256 + 16 * c) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ void to_float(float f[8]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = __uint_as_float(a[i]);
            f[4 + i] = __uint_as_float(b[i]);
        }
    }
    __device__ __forceinline__ float dot(const RowSlice& o) const {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) d = fmaf(__uint_as_float(a[i]), __uint_as_float(o.a[i]), d);
#pragma unroll
        for (int i = 0; i < 4; ++i) d = fmaf(__uint_as_float(b[i]), __uint_as_float(o.b[i]), d);
        return d;
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
constexpr float kLazyMax = 8.0f;

// K and V rows of one page held by a lane: page rows rg, rg+4, rg+8, rg+12.
template <typename E>
struct PageRegs {
    RowSlice<E> k[4], v[4];
};

// P.V of one page for one query head: acc[e] += sum_j p[j] v[j][e] over the
// lane's four rows j, and l += sum_j p[j].  16-bit storage: V rows are
// regrouped into (row 2h, row 2h+1) pairs of each dim with v_perm_b32 once
// per page (prep), P is rounded to the storage type, and each dim takes two
// dot2 instructions; the row sum adds the same rounded P.  f32: FMAs.
template <typename E>
struct PagePV {
    uint32_t lo[2][4], hi[2][4];  // row pair h, dim pair i: (v[2h][2i], v[2h+1][2i]) and (.. [2i+1])
    __device__ __forceinline__ void prep(const RowSlice<E> (&v)[4]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[h][i] = __builtin_amdgcn_perm(v[2 * h + 1].w[i], v[2 * h].w[i], 0x05040100u);
                hi[h][i] = __builtin_amdgcn_perm(v[2 * h + 1].w[i], v[2 * h].w[i], 0x07060302u);
            }
        }
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b);
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
    __device__ __forceinline__ void accumulate(const float p[4], float acc[8], float& l) const {
        const uint32_t p01 = pack2(p[0], p[1]), p23 = pack2(p[2], p[3]);
        l = dot2(p23, kOnes, dot2(p01, kOnes, l));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] = dot2(lo[1][i], p23, dot2(lo[0][i], p01, acc[2 * i]));
            acc[2 * i + 1] = dot2(hi[1][i], p23, dot2(hi[0][i], p01, acc[2 * i + 1]));
        }
    }
    static constexpr uint32_t kOnes = std::is_same<E, BF16>::value ? 0x3f803f80u : 0x3c003c00u;  // (1, 1)
};
template <>
__device__ __forceinline__ uint32_t PagePV<BF16>::pack2(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)a, (__bf16)b});
}
template <>
__device__ __forceinline__ float PagePV<BF16>::dot2(uint32_t a, uint32_t b, float c) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}
template <>
__device__ __forceinline__ uint32_t PagePV<F16>::pack2(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}
template <>
__device__ __forceinline__ float PagePV<F16>::dot2(uint32_t a, uint32_t b, float c) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}
template <>
struct PagePV<F32> {
    float vf[4][8];
    __device__ __forceinline__ void prep(const RowSlice<F32> (&v)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j].to_float(vf[j]);
    }
    __device__ __forceinline__ void accumulate(const float p[4], float acc[8], float& l) const {
        l += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float t = acc[e];
            t = fmaf(p[0], vf[0][e], t);
            t = fmaf(p[1], vf[1][e], t);
            t = fmaf(p[2], vf[2][e], t);
            t = fmaf(p[3], vf[3][e], t);
            acc[e] = t;
        }
    }
};

__device__ __forceinline__ int pages_of(int kv_len) { return kv_len > 0 ? (kv_len + kPage - 1) / kPage : 0; }

// Keys seen by sequence b's query and the row of q / out that holds it.  A
// decode call: kv_lens[b] keys, row b.  Decode rows of a varlen prefill call
// (cu_seqlens set): a sequence of exactly one token t = cu_seqlens[b] sees
// keys j < kv_lens[b] with j <= positions[t] (the prefill kernel's causal
// rule); every other sequence is left to the prefill kernel (no keys here).
__device__ __forceinline__ bool decode_row_of(const DecodeArgs& a, int b, int& row, int& len) {
    if (!a.cu_seqlens) {
        row = b;
        len = a.kv_lens[b];
        return true;
    }
    row = a.cu_seqlens[b];
    if (a.cu_seqlens[b + 1] - row != 1) {
        len = 0;
        return false;
    }
    const int kvl = a.kv_lens[b];
    const int pos = a.positions[row];
    len = pos < kvl ? max(0, pos + 1) : kvl;
    return true;
}
__device__ __forceinline__ int decode_len(const DecodeArgs& a, int b) {
    int row, len;
    decode_row_of(a, b, row, len);
    return len;
}

// Softmax state of query heads h0 .. h0+NREP-1 of sequence b over pages
// [lp0, lp0 + n) of its kv_len keys (query row qrow): the running max m
// (log2 units), the row sum l and the 8 unnormalised accumulators of this
// lane's dims.  On return every lane holds the state of the whole wave for
// its dims (lane & 15).  Used by the split workers (one segment of a slice)
// and by the one-launch kernel (a quarter of a sequence per wave).
//
// FULL: head_dim == 128 (every lane reads its 8 dims); else a.head_dim < 128
// and lanes read only the dims below it (the rest are zeros).
template <typename E, int NREP, bool FULL = true>
__device__ __forceinline__ void decode_segment(const DecodeArgs& a, int b, int kv_len, int lp0, int n, int qrow,
                                               int h0, int64_t head_off, float (&m)[NREP], float (&l)[NREP],
                                               float (&acc)[NREP][8]) {
    constexpr int EB = E::kBytes;
    const int lane = threadIdx.x & 63;
    const int rg = lane >> 4;
    const int c = lane & 15;
    const char* qbase = reinterpret_cast<const char*>(a.q);
    const char* kpool = reinterpret_cast<const char*>(a.k_pool);
    const char* vpool = reinterpret_cast<const char*>(a.v_pool);
    RowSlice<E> qs[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r)
    {
        const char* qr = qbase + ((int64_t)(h0 + r) * a.q_stride_head + (int64_t)qrow * a.q_stride_seq) * EB;
        if constexpr (FULL) qs[r].load(qr, c);
        else qs[r].load_d(qr, c, a.head_dim);
    }
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
            if constexpr (FULL) {
                pr.k[j].stream(kpool + off, c);
                pr.v[j].stream(vpool + off, c);
            } else {
                pr.k[j].stream_d(kpool + off, c, a.head_dim);
                pr.v[j].stream_d(vpool + off, c, a.head_dim);
            }
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
#pragma unroll
            for (int r = 0; r < NREP; ++r) sc[r][j] = pr.k[j].dot(qs[r]);
        }
        // Raw scores (unscaled; the scale folds into the exponentials).
        // Rows past kv_len only occur on a sequence's last page.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) sc[r][j] = row16_sum(sc[r][j]);
        }
        if (pg * kPage + kPage > kv_len) {  // wave-uniform
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool valid = (pg * kPage + rg + 4 * j) < kv_len;
#pragma unroll
                for (int r = 0; r < NREP; ++r) sc[r][j] = valid ? sc[r][j] : -INFINITY;
            }
        }
        // Lazy rescale: the running max m (log2 units) only moves when a
        // page's max exceeds it by more than kLazyMax, so exponentials
        // stay <= 2^kLazyMax and the accumulators are rarely rescaled.
        const float scale = a.scale_log2;
        auto page_max = [&](int r) {
            return fmaxf(fmaxf(sc[r][0], sc[r][1]), fmaxf(sc[r][2], sc[r][3])) * scale;
        };
        bool grow = false;
#pragma unroll
        for (int r = 0; r < NREP; ++r) grow |= page_max(r) > m[r] + kLazyMax;
        if (__ballot(grow)) {
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                const float mn = fmaxf(m[r], page_max(r));
                const float al = fast_exp2(m[r] - mn);
                l[r] *= al;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r][e] *= al;
                m[r] = mn;
            }
        }
        PagePV<E> pv;
        pv.prep(pr.v);
#pragma unroll
        for (int r = 0; r < NREP; ++r) {
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = fast_exp2(fmaf(sc[r][j], scale, -m[r]));
            pv.accumulate(p, acc[r], l[r]);
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
}

// Load-balanced split-KV decode.  Every wave is an independent worker: the
// pages of all sequences are concatenated (per KV head group) and cut into
// equal slices of C pages, one slice per wave, with as many waves as the GPU
// holds at once.  A wave walks its slice sequence by sequence and leaves one
// partial softmax state per (sequence segment, query head); the merge kernel
// combines them.  Slice s of sequence b is partial slot s - first_wave(b).
// The waves of workgroup `block` (4 per workgroup, no barriers: a wave may
// return on its own); used by the decode kernel and by the fused prefill
// launch, whose first workgroups are decode workers.
template <typename E, int NREP, bool FULL = true>
__device__ __forceinline__ void decode_waves(const DecodeArgs& a, int block) {
    const int lane = threadIdx.x & 63;
    const int gw = block * 4 + (threadIdx.x >> 6);
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
        const int pg = pages_of(decode_len(a, i));
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
        my_len = i < B ? decode_len(a, i) : 0;
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

    const int64_t head_off = (int64_t)kvh * a.pool_stride_head;
    const int H = a.n_heads;

    int x = x0;
    while (x < x1) {
        if (b - base >= kWave) {  // next chunk of sequences
            carry += chunk_total;
            base += kWave;
            const int i = base + lane;
            my_len = i < B ? decode_len(a, i) : 0;
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

        const int qrow = a.cu_seqlens ? a.cu_seqlens[b] : b;
        float m[NREP], l[NREP], acc[NREP][8];
        decode_segment<E, NREP, FULL>(a, b, kv_len, lp0, n, qrow, h0, head_off, m, l, acc);

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

}  // namespace femto
