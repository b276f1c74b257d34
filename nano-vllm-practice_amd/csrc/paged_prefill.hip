// Chunked / varlen / causal paged prefill attention and dense flash
// attention on gfx950 MFMA (v_mfma_f32_32x32x16_{bf16,f16}).
//
// Semantics: token t of sequence b (cu_seqlens[b] <= t < cu_seqlens[b+1])
// attends key j iff j < kv_lens[b] and j <= positions[t]
// (femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:83-120 and
// csrc/paged_attention/paged_attention_gemm.cu:179-184 of the reference);
// key j lives at pool[tables[b][j / 16], h / n_rep, j % 16].  The dense
// entry (csrc/flash_attention/flash_attention_warp.cu:20-299) is the same
// contraction with contiguous keys and no causal limit.
//
// Work decomposition:
//  * a workgroup (4 waves) owns G query heads that share one KV head and a
//    block of BT = 32 * 4 / G tokens; each wave owns 32 tokens of one head,
//    so K/V tiles staged in LDS are used by 4 x 32 query rows;
//  * KV is consumed in tiles of 64 keys (4 pages), double-buffered in LDS.
//    Both K and V are copied HBM -> LDS with global_load_lds_dwordx4 (no
//    VGPR staging, no VALU), wave w fetching page w of the tile.  Rows are
//    kept row-major [key][dim] with 16-byte chunks XOR-swizzled by row, so
//    the K operand reads (ds_read_b128) and the transposed V operand reads
//    (ds_read_b64_tr_b16) are bank-conflict free.  A tile's copies go out
//    in one burst after the tile barrier, except in launches whose decode
//    workers have one-token sequences to run: there they are issued one per
//    score MFMA pair, so they do not hold up the workers' page loads;
//  * per tile and wave: S^T(64 x 32) = K . Q^T with 16 MFMAs (Q stays in
//    registers as the B operand), online softmax with the query index equal
//    to the lane (mod 32), then O^T(128 x 32) += V^T . P^T with 16 MFMAs, P
//    taken straight from the S^T accumulators, rounded to the storage type
//    (the reference's Triton kernel rounds P the same way, line 153-155);
//  * causal tile skipping: a wave skips tiles past its largest visible key
//    and applies the mask only on tiles that cross its smallest limit; the
//    running max moves lazily (only when a row max grows by > 2^8), so O is
//    rarely rescaled;
//  * tiles of one sequence are issued heaviest (last) first, and the work
//    list is laid out so each XCD (workgroup id mod 8) gets a contiguous
//    range of KV heads, keeping a head's pages in one L2;
//  * key split (paged, when the caller gives a workspace): a query tile
//    whose sequence is much longer than the average work per resident
//    workgroup is cut into P <= 8 pieces over its key tiles, so one long
//    sequence no longer sets the length of the whole call; only when all
//    pieces fit in the resident workgroup slots at once.  Every piece
//    writes its partial (m, l, O) with system-scope stores (written through
//    to memory), waits for them, and counts itself in with a device-scope
//    atomic; the piece that arrives last reads the others' partials with
//    system-scope loads, merges them into its registers and writes the
//    output.  Only the partials bypass the caches, so no cache-wide
//    write-back or invalidate is needed.  The last piece also resets the
//    counter, leaving the counters all zero; a slot is always written in
//    the call that reads it, so the slots need no clearing.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "decode_worker.h"
#include "launch.h"

namespace femto {

constexpr int kKvTile = 64;
constexpr int kStages = 2;
constexpr int kRowBytes = kDimHead * 2;                // 256
constexpr int kTileBytes = kKvTile * kRowBytes;        // 16 KB per K or V tile
constexpr float kEmptyMaxP = -1.0e30f;
constexpr int kSplitTries = 4;  // key-split granularities tried (T grows by half each time)

// One page of zeros: the source of every copy whose block id lies outside
// the pool (each of its rows is read from row 0), so such a page reads as
// zeros.
__device__ __attribute__((aligned(16))) uint16_t g_zero_page[kPage * kDimHead];

// 16-byte chunk c of LDS row r lives at chunk position c ^ swz(r).  The V
// swizzle gives the four rows that one transposed read covers (r % 4 = 0..3)
// four XOR values that differ in bits 1-2 and in bits 2-3, and the next four
// rows the same values with bit 0 flipped, so the 16-lane groups of a
// ds_read_b64_tr_b16 spread over all banks (measured 282 vs 244 B/ns per CU
// with (r % 8) << 1).
__device__ __forceinline__ int swz_k(int r) { return r & 15; }
__device__ __forceinline__ int swz_v(int r) { return ((r & 1) ? 6 : 0) ^ ((r & 2) ? 10 : 0) ^ ((r & 4) ? 1 : 0); }

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// 16 bytes per lane from global memory (uniform base + per-lane offset)
// straight into LDS at lds_base + 16 * lane.  Issued through asm so the
// compiler does not order later LDS reads of the other stage behind it; the
// kernel waits for these copies itself (vmcnt) before the stage is read.
// base and lds_base must be the same in every lane of the wave.  m0 is on the
// clobber list; clang warns that it is reserved, but nothing else in these
// kernels uses m0 (their assembly sets it only here), so the warning is muted.
//
// The compiler inserts no hazard wait states inside inline asm, so the block
// carries the two that gfx9 requires here: a VMEM instruction may read an
// SGPR only 5 wait states after a VALU instruction wrote it (the base and the
// m0 value usually come straight from v_readfirstlane), and an LDS DMA may
// read m0 only 1 wait state after an SALU instruction wrote it.  Without them
// a copy can use a stale base register and read from a wrong address.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint64_t wave_base(const void* base) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// One page of K and one of V: four copies of each, the copy j of K landing
// at kd + 1024 j and of V at vd + 1024 j.  All eight go out from one asm
// block, so the 5 wait states after the SGPR writes are paid once; each m0
// step (an SALU write) is followed by the 1 wait state the DMA needs.
__device__ __forceinline__ void lds_dma_page(const void* kbase, const void* vbase, const uint32_t (&ko)[4],
                                             const uint32_t (&vo)[4], uint32_t kd, uint32_t vd) {
    const uint64_t kb = wave_base(kbase), vb = wave_base(vbase);
    const uint32_t km0 = __builtin_amdgcn_readfirstlane(kd);
    const uint32_t vm0 = __builtin_amdgcn_readfirstlane(vd);
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 m0, %10\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %8\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %8\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %8\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %3, %8\n\t"
        "s_mov_b32 m0, %11\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %4, %9\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %5, %9\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %6, %9\n\t"
        "s_add_u32 m0, m0, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %7, %9"
        :
        : "v"(ko[0]), "v"(ko[1]), "v"(ko[2]), "v"(ko[3]), "v"(vo[0]), "v"(vo[1]), "v"(vo[2]), "v"(vo[3]),
          "s"(kb), "s"(vb), "s"(km0), "s"(vm0)
        : "memory", "m0", "scc");
}
// One copy of the same kind, for copies issued one at a time between other
// instructions (same wait states as above).
__device__ __forceinline__ void lds_dma_one(uint64_t base_in, uint32_t off, uint32_t m0_in) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base_in);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base_in >> 32));
    const uint64_t base = ((uint64_t)hi << 32) | lo;
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(m0_in);
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(off), "s"(base), "s"(m0v)
        : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// System-scope 16-byte accesses of the key-split partials (buffer
// instructions with sc0 sc1: written through to memory, read past the caches).
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, kPartSlotBytes, 0x00020000);
}
__device__ __forceinline__ void sys_store16(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, v), r, off, 0, 0x11);
}
__device__ __forceinline__ f32x4 sys_load16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0x11));
}

// Sums of N values over the workgroup (every thread gets them); s_red holds 4 * N ints.
template <int N>
__device__ __forceinline__ void block_reduce_n(int (&v)[N], int* s_red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = wave_sum_i32(v[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < N; ++k) s_red[4 * k + wave] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = s_red[4 * k] + s_red[4 * k + 1] + s_red[4 * k + 2] + s_red[4 * k + 3];
    __syncthreads();
}

// Inclusive workgroup scan (every thread gets its prefix and the total);
// s_red holds 4 ints.
__device__ __forceinline__ int block_incl_scan(int v, int* s_red, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_incl_scan_i32(v);
    if (lane == 63) s_red[wave] = v;
    __syncthreads();
    int off = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int x = s_red[w];
        off += (w < wave) ? x : 0;
        total += x;
    }
    __syncthreads();
    return v + off;
}

// Position in an XCD's stretch of the work list of the k-th workgroup the
// XCD receives: the first `cus` workgroups take one slot on each of its CUs,
// the next `cus` the second slot, and so on.  Every other round is dealt in
// reverse, so a CU whose first item is one of the heaviest of the stretch
// (a sequence's items come heaviest first) gets one of the lightest as its
// second; the heavy item then runs alone once the light one is done.
__device__ __forceinline__ int serpentine(int k, int n, int cus) {
    if (cus <= 0) return k;
    const int round = k / cus, pos = k - round * cus;
    if ((round & 1) == 0) return k;
    const int in_round = min(cus, n - round * cus);
    return round * cus + (in_round - 1 - pos);
}

// FULLD: head_dim == 128.  Else (paged calls only) head_dim is a smaller
// multiple of 16 and the tile loop is the same code: K and V rows keep
// their 256-byte LDS slots, and lanes whose 16-byte chunk lies at or past
// head_dim copy chunk 0 of the same row instead (in bounds, finite for
// finite pools); Q is zero past head_dim, so those K dims add nothing to the
// scores; the V dims past head_dim only reach output dims that are not
// stored.  The MFMAs past head_dim are spent for nothing: such calls run
// at the speed of head_dim 128.
template <typename E, int G, bool PAGED, bool FUSED, bool FULLD = true>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_mfma_kernel(PrefillArgs a) {
    constexpr int EB = 2;
    constexpr int BT = 32 * (4 / G);
    // [stage][0 = K, 1 = V][64 keys x 256 B]
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages][2][kTileBytes];
    __shared__ int s_red[4 * (kSplitTries + 2)];
    __shared__ int s_seq, s_ltile, s_old;
    __shared__ int s_kend[4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
    const int l32 = lane & 31;
    const int h2 = lane >> 5;

    // ---- work item, XCD-aware: workgroup id mod 8 selects the XCD, and
    // each XCD takes a contiguous range of the work list (KV head groups
    // outermost, so a head's pages stay in one L2).
    int lin = blockIdx.x;
    if constexpr (FUSED) {
        // The first workgroups are decode workers (G query heads per wave, as
        // the decode kernel would use for this head ratio); they are
        // dispatched first, one per CU, and the tiles fill the other slots.
        if (lin < a.decode_blocks) {
            decode_waves<E, G, FULLD>(a.dec, lin);
            return;
        }
        lin -= a.decode_blocks;  // a multiple of 8: the XCD of a tile is unchanged
    }
    int grp, tile_lin;
    int b, tile, q_begin, q_end, kv_len;
    // Key split of this query tile: piece `piece` of `npieces`; its siblings
    // are work items sib_base + p * sib_stride (piece-major order), which
    // also index their partial slots; the counter is piece 0's.
    int piece = 0, npieces = 1, sib_base = 0, sib_stride = 0;
    // Copies issued one per score MFMA pair instead of in one burst (only in
    // a launch whose decode workers have one-token sequences to run).
    bool spread = false;
    if constexpr (PAGED) {
        const int groups = a.n_kv_heads * a.head_groups;
        bool split = a.part != nullptr;
        // Per-sequence sizes, loaded once: thread t keeps sequence t (the
        // passes below reload only for sequences past the first 256).
        int my_q0 = 0, my_ql = 0, my_kvl = 0, my_dec = 0;
        if (tid < a.num_seqs) {
            my_q0 = a.cu_seqlens[tid];
            my_ql = a.cu_seqlens[tid + 1] - my_q0;
            my_dec = a.skip_decode_rows && my_ql == 1;
            if (my_dec) my_ql = 0;  // run by the decode kernel
            my_kvl = a.kv_lens[tid];
        }
        auto seq_sizes = [&](int i, int& ql, int& kvl) {
            if (i < 256) {
                ql = my_ql;
                kvl = my_kvl;
            } else {
                ql = a.cu_seqlens[i + 1] - a.cu_seqlens[i];
                if (a.skip_decode_rows && ql == 1) ql = 0;
                kvl = a.kv_lens[i];
            }
        };
        // Pieces per query tile of sequence i: round(key tiles / T), at most
        // kMaxPieces, where T0 is the estimated key tiles per resident
        // workgroup of the whole call (query tile j of a chunk of ql tokens
        // sees about kv_len - ql + BT (j+1) keys).  A sequence up to 1.5 times
        // the average is not split.
        int T0 = 0;
        if (split) {
            for (int base = 0; base < a.num_seqs; base += 256) {
                const int i = base + tid;
                int est = 0;
                if (i < a.num_seqs) {
                    int ql, kvl;
                    seq_sizes(i, ql, kvl);
                    if (ql > 0 && kvl > 0) {
                        const int mean_keys = min(kvl, max(1, kvl - ql + (ql + BT) / 2));
                        est = ((ql + BT - 1) / BT) * ((mean_keys + kKvTile - 1) / kKvTile);
                    }
                }
                int tot[1] = {est};
                block_reduce_n(tot, s_red);
                T0 += tot[0];
            }
            T0 = max(8, (int)(((int64_t)T0 * groups + a.resident - 1) / a.resident));
        }
        // Pieces only pay off in workgroup slots that would otherwise idle
        // (a second round of pieces costs more than it balances): of the
        // candidates T0, 1.5 T0, 2.25 T0, 3.375 T0 (fewer sequences split
        // each time) the first whose pieces all fit in the resident slots at
        // once is taken, else the call runs unsplit.
        int w = 0;
        if (tid == 0) s_seq = -1;
        if (!split && a.num_seqs <= 256) {
            // Unsplit call, one sequence per thread: a single scan gives both
            // the work total and each sequence's first query tile.
            const int nt = tid < a.num_seqs && my_ql > 0 ? (my_ql + BT - 1) / BT : 0;
            // beside decode workers with one-token sequences the copies are spread
            if constexpr (FUSED) spread = __syncthreads_or(my_dec) != 0;
            int total;
            const int incl = block_incl_scan(nt, s_red, total);
            const int work = groups * total;
            const int per_xcd = (work + 7) >> 3;
            if ((lin >> 3) >= per_xcd) return;
            w = (lin & 7) * per_xcd + serpentine(lin >> 3, per_xcd, a.resident >> 4);
            if (w >= work) return;
            grp = w / total;
            tile_lin = w - grp * total;
            if (nt > 0 && tile_lin >= incl - nt && tile_lin < incl) {
                s_seq = tid;
                s_ltile = tile_lin - (incl - nt);
                s_kend[0] = my_q0;  // q_begin (s_kend is rewritten below)
                s_kend[1] = my_ql;
                s_kend[2] = my_kvl;
                s_kend[3] = 1;
            }
        } else {
            int Tk[kSplitTries];
            Tk[0] = T0;
#pragma unroll
            for (int k = 1; k < kSplitTries; ++k) Tk[k] = Tk[k - 1] + Tk[k - 1] / 2;
            auto pieces_of = [&](int kvl, int t) {
                const int ub = kvl > 0 ? (kvl + kKvTile - 1) / kKvTile : 0;
                return min(kMaxPieces, max(1, (2 * ub + t) / (2 * t)));
            };
            // pieces per KV head group for each T, then unsplit, then the
            // sequences the decode workers run
            int cnt[kSplitTries + 2] = {};
            for (int base = 0; base < a.num_seqs; base += 256) {
                const int i = base + tid;
                int c[kSplitTries + 2] = {};
                if (i < a.num_seqs) {
                    int ql, kvl;
                    seq_sizes(i, ql, kvl);
                    const int nt = ql > 0 ? (ql + BT - 1) / BT : 0;
#pragma unroll
                    for (int k = 0; k < kSplitTries; ++k) c[k] = split ? nt * pieces_of(kvl, Tk[k]) : nt;
                    c[kSplitTries] = nt;
                    if constexpr (FUSED)
                        c[kSplitTries + 1] = i < 256 ? my_dec : (a.cu_seqlens[i + 1] - a.cu_seqlens[i] == 1);
                }
                block_reduce_n(c, s_red);
#pragma unroll
                for (int k = 0; k <= kSplitTries + 1; ++k) cnt[k] += c[k];
            }
            if constexpr (FUSED) spread = __builtin_amdgcn_readfirstlane(cnt[kSplitTries + 1]) > 0;
            int T = 0, total = cnt[kSplitTries];
            if (split) {
#pragma unroll
                for (int k = kSplitTries - 1; k >= 0; --k) {
                    if ((int64_t)groups * cnt[k] <= a.resident) {
                        T = Tk[k];
                        total = cnt[k];
                    }
                }
            }
            split = T > 0;
            const int work = groups * total;
            const int per_xcd = (work + 7) >> 3;
            if ((lin >> 3) >= per_xcd) return;
            w = (lin & 7) * per_xcd + (split ? (lin >> 3) : serpentine(lin >> 3, per_xcd, a.resident >> 4));
            if (w >= work) return;
            grp = w / total;
            tile_lin = w - grp * total;

            // The sequence of piece tile_lin.  Within a sequence come first the
            // first pieces of all its query tiles (heaviest, i.e. last, tile
            // first), then the second pieces, and so on: lengths fall smoothly
            // along the dispatch order, so no run of long pieces queues behind
            // one shader engine while others idle.
            int carry = 0;
            for (int base = 0; base < a.num_seqs; base += 256) {
                const int i = base + tid;
                int nt = 0, pp = 1, ql = 0, kvl = 0;
                if (i < a.num_seqs) {
                    seq_sizes(i, ql, kvl);
                    nt = ql > 0 ? (ql + BT - 1) / BT : 0;
                    pp = split ? pieces_of(kvl, T) : 1;
                }
                int tot;
                const int incl = block_incl_scan(nt * pp, s_red, tot);
                const int excl = incl - nt * pp;
                if (i < a.num_seqs && tile_lin >= carry + excl && tile_lin < carry + incl) {
                    s_seq = i;
                    s_ltile = tile_lin - carry - excl;
                    s_kend[0] = i < 256 ? my_q0 : a.cu_seqlens[i];  // q_begin (s_kend is rewritten below)
                    s_kend[1] = ql;
                    s_kend[2] = kvl;
                    s_kend[3] = pp;
                }
                carry += tot;
                if (carry > tile_lin) break;
            }
        }
        __syncthreads();
        b = s_seq;
        if (b < 0) return;
        q_begin = s_kend[0];
        q_end = q_begin + s_kend[1];
        kv_len = s_kend[2];
        npieces = s_kend[3];
        const int nt = (s_kend[1] + BT - 1) / BT;
        piece = s_ltile / nt;
        const int jh = s_ltile - piece * nt;
        tile = nt - 1 - jh;  // heaviest tile of the sequence first
        sib_base = w - s_ltile + jh;
        sib_stride = nt;
        __syncthreads();  // s_kend is reused below
    } else {
        const int per_xcd = (int)gridDim.x >> 3;
        const int w = (lin & 7) * per_xcd + (lin >> 3);
        if (w >= a.total_work) return;
        grp = w / a.tiles_per_group;
        tile_lin = w - grp * a.tiles_per_group;
        const int tpb = (a.q_len + BT - 1) / BT;
        b = tile_lin / tpb;
        tile = tile_lin - b * tpb;
        q_begin = 0;
        q_end = a.q_len;
        kv_len = a.kv_len;
    }
    const int kvh = grp / a.head_groups;
    const int hg = grp - kvh * a.head_groups;

    const int hw = wave % G;
    const int tb = wave / G;
    const int h = kvh * a.n_rep + hg * G + hw;
    const int t = q_begin + tile * BT + tb * 32 + l32;  // this lane's query token
    const bool qvalid = t < q_end;

    // ---- KV staging: wave w copies page w of each tile (16 keys x 256 B of
    // K and of V) with 4 + 4 direct-to-LDS loads; in load j, lane i writes
    // LDS row 16w + 4j + i/16, chunk position i%16, and so fetches logical
    // chunk (i%16) ^ swz(row).
    const char* kbase_p = reinterpret_cast<const char*>(a.k);
    const char* vbase_p = reinterpret_cast<const char*>(a.v);
    const int32_t* table = PAGED ? a.tables + (int64_t)b * a.table_stride : nullptr;
    const int npages_tbl = PAGED ? min(a.num_pages_per_seq, (kv_len + kPage - 1) / kPage) : 0;
    const int lrow = lane >> 4;  // row within the load's group of 4
    const int lpos = lane & 15;
    // Byte offsets of this lane's chunks: inside its row (koff, voff) and
    // inside a full page of the pool (kfull, vfull, rows 4j + lrow).  The
    // copies of a full tile use the precomputed page offsets, so the issue
    // path does no address arithmetic that could tie it to a pending load.
    const int rs_k = (int)a.k_stride2 * EB, rs_v = (int)a.v_stride2 * EB;
    int koff[4], voff[4];
    uint32_t kfull[4], vfull[4];
    const int nchunks = FULLD ? 16 : a.head_dim / 8;  // 16-byte chunks per row
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + lrow;
        const int ck = lpos ^ swz_k(r), cv = lpos ^ swz_v(r);
        koff[j] = ((FULLD || ck < nchunks) ? ck : 0) << 4;
        voff[j] = ((FULLD || cv < nchunks) ? cv : 0) << 4;
        kfull[j] = (uint32_t)(r * rs_k + koff[j]);
        vfull[j] = (uint32_t)(r * rs_v + voff[j]);
    }
    // Block ids for this wave's page of tiles tbase .. tbase+63, one per lane.
    int tbl = -1, tbase = 0;
    auto fetch_table = [&](int it0) __attribute__((always_inline)) {
        tbase = it0;
        const int pg = 4 * (it0 + lane) + wave;
        tbl = (PAGED && pg < npages_tbl) ? table[pg] : -1;
    };

    // A tile's copies prepared by issue_tile (prep set) and issued one at a
    // time: copy j < 4 is K rows 4j + lrow, copy 4 + j the same V rows.
    uint64_t pc_kb = 0, pc_vb = 0;
    uint32_t pc_kd = 0, pc_vd = 0, pc_ko[4] = {}, pc_vo[4] = {};
    bool prep = false;
    auto copy_one = [&](int j) __attribute__((always_inline)) {
        if (j < 4) lds_dma_one(pc_kb, pc_ko[j], pc_kd + 1024 * j);
        else lds_dma_one(pc_vb, pc_vo[j - 4], pc_vd + 1024 * (j - 4));
    };
    auto issue_tile = [&](int it, int stage) __attribute__((always_inline)) {
        const int key0 = it * kKvTile + 16 * wave;  // first key of this wave's page
        // Keys past kv_len read the last visible key's row (finite data,
        // masked later); pages wholly past kv_len read that key's page.
        const int kc = key0 < kv_len ? key0 : kv_len - 1;
        const int last_row = kv_len - 1 - (kc & ~15);
        const char* kp;
        const char* vp;
        bool ok = true;
        if constexpr (PAGED) {
            int blk = -1;
            if (key0 < kv_len) {
                blk = __builtin_amdgcn_readlane(tbl, it - tbase);
            } else {
                const int pg = kc >> 4;
                blk = pg < npages_tbl ? table[pg] : -1;
                blk = __builtin_amdgcn_readfirstlane(blk);
            }
            ok = blk >= 0 && (int64_t)blk < a.num_blocks;
            kp = ok ? kbase_p + ((int64_t)blk * a.k_stride0 + (int64_t)kvh * a.k_stride1) * EB
                    : reinterpret_cast<const char*>(g_zero_page);
            vp = ok ? vbase_p + ((int64_t)blk * a.v_stride0 + (int64_t)kvh * a.v_stride1) * EB
                    : reinterpret_cast<const char*>(g_zero_page);
        } else {
            const int k16 = kc & ~15;
            kp = kbase_p + ((int64_t)b * a.k_stride0 + (int64_t)kvh * a.k_stride1 + (int64_t)k16 * a.k_stride2) * EB;
            vp = vbase_p + ((int64_t)b * a.v_stride0 + (int64_t)kvh * a.v_stride1 + (int64_t)k16 * a.v_stride2) * EB;
        }
        const uint32_t kd = lds_addr(&smem[stage][0][(16 * wave) * kRowBytes]);
        const uint32_t vd = lds_addr(&smem[stage][1][(16 * wave) * kRowBytes]);
        if (prep) {  // only the sources and destinations, for copy_one
            const bool full = ok && last_row >= kPage - 1;
            pc_kb = (uint64_t)(uintptr_t)kp;
            pc_vb = (uint64_t)(uintptr_t)vp;
            pc_kd = kd;
            pc_vd = vd;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = ok ? min(4 * j + lrow, last_row) : 0;
                pc_ko[j] = full ? kfull[j] : (uint32_t)(row * rs_k + koff[j]);
                pc_vo[j] = full ? vfull[j] : (uint32_t)(row * rs_v + voff[j]);
            }
            return;
        }
        if (ok && last_row >= kPage - 1) {  // a full page of the pool (wave-uniform)
            lds_dma_page(kp, vp, kfull, vfull, kd, vd);
        } else {
            // The sequence's last page (rows past kv_len repeat its last row)
            // or the zero page (every row reads row 0: all of it is zeros).
            uint32_t ko[4], vo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = ok ? min(4 * j + lrow, last_row) : 0;
                ko[j] = (uint32_t)(row * rs_k + koff[j]);
                vo[j] = (uint32_t)(row * rs_v + voff[j]);
            }
            lds_dma_page(kp, vp, ko, vo, kd, vd);
        }
    };

    // The first tile of this piece does not depend on the causal limits:
    // its block ids and its copy into LDS go out now, while the positions
    // load below is in flight.  Every exit before the tile loop waits for
    // this copy (it must not land in LDS after the workgroup has left).
    int t_first = 0;
    if (PAGED && npieces > 1) {
        const int ub = (kv_len + kKvTile - 1) / kKvTile;
        t_first = piece * ((ub + npieces - 1) / npieces);
    }
    const bool first_issued = t_first * kKvTile < kv_len;
    if (first_issued) {
        fetch_table(t_first);
        issue_tile(t_first, 0);
    }

    // Number of keys visible to this lane's query.
    int lim;
    if constexpr (PAGED) {
        const int pos = qvalid ? a.positions[t] : kv_len;
        lim = pos + 1 < kv_len ? pos + 1 : kv_len;
        lim = lim < 0 ? 0 : lim;
    } else {
        lim = kv_len;
    }
    // Wave-uniform (scalar) limits, so that the tile loop branches on scalars.
    const int kend_w = wave_max_i32(qvalid ? lim : 0);
    const int kfull_w = wave_min_i32(qvalid ? lim : 0x7fffffff);
    if (lane == 0) s_kend[wave] = kend_w;
    __syncthreads();
    const int kend = max(max(s_kend[0], s_kend[1]), max(s_kend[2], s_kend[3]));

    // Key tiles of this piece: [t_lo, t_hi).  Pieces past the query tile's
    // last visible key have nothing to do (and are not counted); a tile that
    // needs a single piece is processed whole.
    const int ntiles = (kend + kKvTile - 1) / kKvTile;
    int t_lo = 0, t_hi = ntiles, nne = 1;
    if (PAGED && npieces > 1) {
        const int ub = (kv_len + kKvTile - 1) / kKvTile;
        const int tp = (ub + npieces - 1) / npieces;
        nne = max(1, (ntiles + tp - 1) / tp);
        if (piece >= nne) {
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the first tile's copy has landed
            return;
        }
        t_lo = piece * tp;
        t_hi = min(ntiles, t_lo + tp);
    }
    if (t_hi <= t_lo) __builtin_amdgcn_s_waitcnt(0x0f70);  // no tile: only wait for the copy

    // Q rows in registers: the B operand of S^T = K . Q^T.
    u32x4 qreg[8];
    {
        const char* qrow = reinterpret_cast<const char*>(a.q) +
                           ((int64_t)b * a.q_stride_batch + (int64_t)h * a.q_stride_head + (int64_t)t * a.q_stride_token) * EB;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            qreg[kk] = (qvalid && (FULLD || 16 * kk < a.head_dim)) ? ld16(qrow + (16 * kk + 8 * h2) * EB)
                                                                  : u32x4{0, 0, 0, 0};
    }

    // Per-lane constant parts of the LDS operand addresses.
    const int k_rd = l32 * kRowBytes;  // K row l32 (+ 32 * kb2 rows)
    const int k_sw = swz_k(l32);
    // V^T operand via ds_read_b64_tr_b16: in each 16-lane group, lane i
    // supplies keys (.. + i/4) x dims (.. + 4*(i%4)); lane j then holds dim j.
    const int gi = lane & 15;
    const int v_key = 4 * h2 + (gi >> 2);                 // + 16*ks + 8*half
    const int v_dim = 16 * ((lane >> 4) & 1) + 4 * (gi & 3);  // + 32*dt

    f32x16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] = f32x16{};
    float m_run = kEmptyMaxP;
    float l_run = 0.0f;
    const float scale = a.scale_log2;

    // One 64-key tile from LDS stage STAGE (a compile-time constant, so the
    // stage offset folds into the LDS instructions' immediate offsets).
    auto tile_math = [&](int kb, auto stage_c, auto copies_c) __attribute__((always_inline)) {
        constexpr int STAGE = decltype(stage_c)::value;
        // copies_c: std::false_type (no copies here), or a bool: issue the
        // next tile's copies between the score MFMAs
        constexpr bool kMayCopy = !std::is_same<decltype(copies_c), std::false_type>::value;
        const uint8_t* ks = smem[STAGE][0];
        const uint8_t* vs = smem[STAGE][1];

        // S^T blocks: keys kb + 32*kb2 + (0..31), queries = lanes (raw scores).
        // The two blocks' MFMA chains alternate, and the K fragments of step
        // kk are read at step kk - 2, so an MFMA does not wait out a full LDS
        // read latency (with one chain after the other and one fragment
        // register, every MFMA of the first chain did).
        f32x16 sacc[2] = {f32x16{}, f32x16{}};
        auto kfrag = [&](int kk, int kb2) {
            const int chunk = (2 * kk + h2) ^ k_sw;
            return *reinterpret_cast<const u32x4*>(ks + k_rd + kb2 * 32 * kRowBytes + (chunk << 4));
        };
        u32x4 kf[3][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            kf[kk][0] = kfrag(kk, 0);
            kf[kk][1] = kfrag(kk, 1);
        }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            if (kk + 2 < 8) {
                kf[(kk + 2) % 3][0] = kfrag(kk + 2, 0);
                kf[(kk + 2) % 3][1] = kfrag(kk + 2, 1);
            }
            sacc[0] = mfma32x32x16(E{}, kf[kk % 3][0], qreg[kk], sacc[0]);
            sacc[1] = mfma32x32x16(E{}, kf[kk % 3][1], qreg[kk], sacc[1]);
            if constexpr (kMayCopy) {
                if (copies_c) copy_one(kk);  // the next tile's copy kk
            }
        }
        // Keep that order: 4 reads, then 6 x (2 reads, 2 MFMAs), then 4 MFMAs.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int g = 0; g < 6; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        // Accumulator i of block kb2 holds key kb + 32*kb2 + 8*(i/4) + 4*h2 + i%4.
        float mx = -INFINITY;
        if (kb + kKvTile > kfull_w) {  // wave-uniform: tile crosses some row's limit
            const int kr = lim - kb - 4 * h2;  // key index relative to this lane's base
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rel = 32 * kb2 + 8 * (i >> 2) + (i & 3);
                    const float s = rel < kr ? sacc[kb2][i] : -INFINITY;
                    sacc[kb2][i] = s;
                    mx = fmaxf(mx, s);
                }
            }
        } else {
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kb2][i]);
            }
        }
        {
            float m_lo, m_hi;  // the row's two lane halves (keys 4*h2 + ...)
            pair32(mx, m_lo, m_hi);
            mx = fmaxf(m_lo, m_hi) * scale;
        }
        // Lazy rescale: the running max m_run only moves when some row's
        // max exceeds it by more than 8 (log2 units), so exponentials stay
        // <= 2^8 and O is rarely rescaled.
        if (__ballot(mx > m_run + 8.0f)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = fast_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;
        }
        const float neg_m = -m_run;

        // P^T as the B operand: k-slot j of lane half h2 in step ks is key
        // kb + 16*ks + 8*(j/4) + 4*h2 + j%4.  The row sum adds the rounded
        // P values the MFMA consumes.
        u32x4 pb[4];
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
            float pf[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pf[j] = fast_exp2(fmaf(sacc[ks2 >> 1][8 * (ks2 & 1) + j], scale, neg_m));
            pb[ks2] = pack8(E{}, pf);
            l_run = sum8(E{}, pb[ks2], l_run);
        }

#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                u32x2 part[2];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int key = 16 * ks2 + 8 * half + v_key;
                    const int dim = 32 * dt + v_dim;
                    const int off = key * kRowBytes + ((((dim >> 3) ^ swz_v(key)) << 4) | ((dim & 4) << 1));
                    const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vs + off));
                    part[half] = __builtin_bit_cast(u32x2, r);
                }
                const u32x4 va = u32x4{part[0][0], part[0][1], part[1][0], part[1][1]};
                oacc[dt] = mfma32x32x16(E{}, va, pb[ks2], oacc[dt]);
            }
        }
    };

    // Loop over tiles two at a time so each half uses a constant stage.
    auto step = [&](int it, auto stage_c, auto spread_c) __attribute__((always_inline)) {
        constexpr int STAGE = decltype(stage_c)::value;
        constexpr bool SPREAD = decltype(spread_c)::value;
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of tile it are in LDS
        __syncthreads();                     // ... and every wave's; the other stage is free again
        const bool more = it + 1 < t_hi;
        if constexpr (SPREAD) {
            // Beside decode workers the next tile's copies go out one per
            // score MFMA pair: a burst of 32 per workgroup holds up the
            // workers' page loads on the CU's address unit (mixed batches
            // 3-5 % faster; calls without decode rows ~10 % slower so).
            if (more) {
                if (((it + 1 - tbase) & ~63) != 0) fetch_table(it + 1);
                prep = true;
                issue_tile(it + 1, STAGE ^ 1);
                prep = false;
            }
        } else if (more) {
            // The copies queue on the CU's address unit; issuing them at
            // raised priority shortens the wave's wait behind the other
            // workgroup's instructions (1-2 % on the prefill workloads).
            __builtin_amdgcn_s_setprio(1);
            if (((it + 1 - tbase) & ~63) != 0) fetch_table(it + 1);
            issue_tile(it + 1, STAGE ^ 1);  // in flight during this tile's math
            __builtin_amdgcn_s_setprio(0);
        }
        const int kb = it * kKvTile;
        if constexpr (SPREAD) {
            if (kb < kend_w) {
                tile_math(kb, stage_c, more);
            } else if (more) {
#pragma unroll
                for (int j = 0; j < 8; ++j) copy_one(j);
            }
        } else {
            if (kb < kend_w) tile_math(kb, stage_c, std::false_type{});
        }
    };
    auto tile_loop = [&](auto spread_c) __attribute__((always_inline)) {
        for (int it = t_lo; it < t_hi; it += 2) {
            step(it, std::integral_constant<int, 0>{}, spread_c);
            if (it + 1 < t_hi) step(it + 1, std::integral_constant<int, 1>{}, spread_c);
        }
    };
    if constexpr (FUSED) {
        if (spread) tile_loop(std::true_type{});
        else tile_loop(std::false_type{});
    } else {
        tile_loop(std::false_type{});
    }

    if (PAGED && nne > 1) {
        // Partial of this piece, lane-major so each lane later reads back
        // exactly its own values.  f32 and f16 storage: the raw accumulators,
        // accumulator k = 4*dt + g of lane l of wave w at
        // 16 * ((16 w + k) * 64 + l), and (m, l) per lane.  bf16 storage:
        // the accumulators divided by the row sum and by a power of two
        // 2^e above their largest magnitude, as fp16 (8 per 16 bytes, chunk
        // k = 2*dt + j at 16 * ((8 w + k) * 64 + l); 2^e as f32 at
        // 32768 + 4 * (64 w + l)), and (m, row sum): half the bytes, which
        // is what a merge costs (one CU reads the other pieces' partials at
        // ~23 GB/s), for an added error of at most 2^-12 of the lane's
        // largest output, below the bf16 output rounding.  (m, l) at
        // 65536 + 8 * (64 w + l) in both layouts.
        // Piece p's slot is its work index sib_base + p * sib_stride (< the
        // resident workgroup count, as split calls have no more pieces).
        constexpr bool kHalf = std::is_same<E, BF16>::value;
        uint8_t* part = reinterpret_cast<uint8_t*>(a.part);
        auto slot_of = [&](int p) { return part + (int64_t)(sib_base + p * sib_stride) * kPartSlotBytes; };
        const int lane_acc = (wave * (kHalf ? 8 : 16) * 64 + lane) * 16;  // + k * 1024
        const int lane_ml = 65536 + (wave * 64 + lane) * 8;
        {
            const auto r = slot_rsrc(slot_of(piece));
            float l_pub = l_run;
            if constexpr (kHalf) {
                float l_lo, l_hi;
                pair32(l_run, l_lo, l_hi);
                l_pub = l_lo + l_hi;
                float amax = 0.0f;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(oacc[dt][e]));
                const float inv = l_pub > 0.0f ? 1.0f / l_pub : 0.0f;
                int ex = 0;
                frexpf(amax * inv, &ex);  // amax * inv < 2^ex
                const float sc = ldexpf(inv, -ex), unsc = ldexpf(1.0f, ex);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        float f[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) f[e] = oacc[dt][8 * j + e] * sc;
                        __builtin_amdgcn_raw_buffer_store_b128(pack8(F16{}, f), r, lane_acc + (2 * dt + j) * 1024, 0,
                                                               0x11);
                    }
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(unsc), r, 32768 + (wave * 64 + lane) * 4, 0, 0x11);
            } else {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        sys_store16(r, lane_acc + (4 * dt + g) * 1024,
                                    f32x4{oacc[dt][4 * g], oacc[dt][4 * g + 1], oacc[dt][4 * g + 2], oacc[dt][4 * g + 3]});
            }
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(m_run), __float_as_uint(l_pub)}, r, lane_ml, 0,
                                                  0x11);
        }
        // The partial is in memory before the count goes up.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int* counter = a.counters + sib_base;
        if (tid == 0) s_old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_old != nne - 1) return;  // another piece merges
        if (tid == 0) __hip_atomic_exchange(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::: "memory");
        // Merge the other pieces' partials, kR per round with all their
        // loads in flight together.  The piece indices are made scalar so
        // the slots' buffer descriptors are scalar (no per-lane descriptor
        // loop around each load), and each round is straight-line code, so
        // it waits for its own loads only.  A round with fewer partials
        // reads its last one again and gives the copies weight 0.
        constexpr int kR = kHalf ? 4 : 2;
        constexpr int kLoads = kHalf ? 8 : 16;
        const int pc = __builtin_amdgcn_readfirstlane(piece);
        const int n_o = __builtin_amdgcn_readfirstlane(nne) - 1;
        const int sb = __builtin_amdgcn_readfirstlane(sib_base);
        const int ss = __builtin_amdgcn_readfirstlane(sib_stride);
        auto other_rsrc = [&](int i) {  // the i-th other piece, this one skipped
            return slot_rsrc(part + (int64_t)(sb + (i < pc ? i : i + 1) * ss) * kPartSlotBytes);
        };
#pragma unroll 1
        for (int i = 0; i < n_o; i += kR) {
            __amdgpu_buffer_rsrc_t r[kR];
            u32x2 ml[kR];
            uint32_t sc[kR];
            u32x4 v[kR][kLoads];
#pragma unroll
            for (int j = 0; j < kR; ++j) {
                r[j] = other_rsrc(min(i + j, n_o - 1));
                ml[j] = __builtin_amdgcn_raw_buffer_load_b64(r[j], lane_ml, 0, 0x11);
                if constexpr (kHalf) sc[j] = __builtin_amdgcn_raw_buffer_load_b32(r[j], 32768 + (wave * 64 + lane) * 4, 0, 0x11);
            }
#pragma unroll
            for (int j = 0; j < kR; ++j)
#pragma unroll
                for (int k = 0; k < kLoads; ++k)
                    v[j][k] = __builtin_amdgcn_raw_buffer_load_b128(r[j], lane_acc + k * 1024, 0, 0x11);
            float m_new = m_run;
#pragma unroll
            for (int j = 0; j < kR; ++j) m_new = fmaxf(m_new, __uint_as_float(ml[j][0]));
            const float al = fast_exp2(m_run - m_new);
            float w[kR], wsum = 0.0f;
#pragma unroll
            for (int j = 0; j < kR; ++j) {
                w[j] = i + j < n_o ? fast_exp2(__uint_as_float(ml[j][0]) - m_new) : 0.0f;
                if constexpr (kHalf) w[j] *= __uint_as_float(ml[j][1]);  // fp16 partials are normalised
                else wsum += w[j] * __uint_as_float(ml[j][1]);
            }
            if constexpr (kHalf) {
#pragma unroll
                for (int j = 0; j < kR; ++j) {
                    wsum += w[j];
                    w[j] *= __uint_as_float(sc[j]);  // undo the partial's power-of-two scale
                }
                // Each half-wave keeps half of the merged pieces' row sum, so
                // the two halves still add up to the row total.
                l_run = l_run * al + 0.5f * wsum;
            } else {
                l_run = l_run * al + wsum;
            }
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[dt][e] *= al;
#pragma unroll
            for (int j = 0; j < kR; ++j) {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    if constexpr (kHalf) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            float f[8];
                            unpack8(F16{}, v[j][2 * dt + h], f);
#pragma unroll
                            for (int e = 0; e < 8; ++e) oacc[dt][8 * h + e] = fmaf(f[e], w[j], oacc[dt][8 * h + e]);
                        }
                    } else {
#pragma unroll
                        for (int g = 0; g < 4; ++g)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                oacc[dt][4 * g + e] = fmaf(__uint_as_float(v[j][4 * dt + g][e]), w[j], oacc[dt][4 * g + e]);
                    }
                }
            }
        }
    }

    // ---- epilogue: O^T accumulator i of dim tile dt holds dim
    // 32*dt + 8*(i/4) + 4*h2 + i%4 of this lane's query.
    float l_lo, l_hi;
    pair32(l_run, l_lo, l_hi);
    const float l_tot = l_lo + l_hi;
    const float inv_l = 1.0f / l_tot;  // 0 visible keys: 1/0 = inf, and 0 * inf = NaN as in the reference
    if (qvalid) {
        char* orow = reinterpret_cast<char*>(a.out) +
                     ((int64_t)b * a.out_stride_batch + (int64_t)h * a.out_stride_head + (int64_t)t * a.out_stride_token) * EB;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * dt + 8 * g + 4 * h2;
                if (!FULLD && d0 >= a.head_dim) continue;  // head_dim is a multiple of 16: d0 + 4 <= head_dim
                const u32x2 v = pack4(E{}, oacc[dt][4 * g] * inv_l, oacc[dt][4 * g + 1] * inv_l,
                                      oacc[dt][4 * g + 2] * inv_l, oacc[dt][4 * g + 3] * inv_l);
                *reinterpret_cast<u32x2*>(orow + d0 * EB) = v;
            }
        }
    }
}

static int pick_group(int n_rep) { return (n_rep % 4 == 0) ? 4 : (n_rep % 2 == 0) ? 2 : 1; }

template <typename E, bool PAGED, bool FUSED, bool FULLD>
static hipError_t launch_gfd(int G, const PrefillArgs& a, hipStream_t st) {
    const int grid = (FUSED ? a.decode_blocks : 0) + ((a.total_work + 7) / 8) * 8;
    switch (G) {
        case 1:
            hipLaunchKernelGGL((attention_mfma_kernel<E, 1, PAGED, FUSED, FULLD>), dim3(grid), dim3(256), 0, st, a);
            break;
        case 2:
            hipLaunchKernelGGL((attention_mfma_kernel<E, 2, PAGED, FUSED, FULLD>), dim3(grid), dim3(256), 0, st, a);
            break;
        case 4:
            hipLaunchKernelGGL((attention_mfma_kernel<E, 4, PAGED, FUSED, FULLD>), dim3(grid), dim3(256), 0, st, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename E, bool PAGED, bool FUSED>
static hipError_t launch_gf(int G, const PrefillArgs& a, hipStream_t st) {
    if (a.head_dim == kDimHead) return launch_gfd<E, PAGED, FUSED, true>(G, a, st);
    if constexpr (PAGED) {
        if (a.head_dim >= 16 && a.head_dim < kDimHead && a.head_dim % 16 == 0)
            return launch_gfd<E, PAGED, FUSED, false>(G, a, st);
    }
    return hipErrorInvalidValue;  // dense attention takes exactly 128
}

template <typename E, bool PAGED>
static hipError_t launch_g(int G, const PrefillArgs& a, hipStream_t st) {
    if constexpr (PAGED) {
        if (a.decode_blocks > 0) return launch_gf<E, true, true>(G, a, st);
    }
    return launch_gf<E, PAGED, false>(G, a, st);
}

template <bool PAGED>
static hipError_t launch_dtype(int dtype, int G, const PrefillArgs& a, hipStream_t st) {
    switch (dtype) {
        case kDtypeBF16: return launch_g<BF16, PAGED>(G, a, st);
        case kDtypeF16: return launch_g<F16, PAGED>(G, a, st);
        default: return hipErrorInvalidValue;
    }
}

// Query tiles per (kv head, head group) are at most num_tokens / BT plus one
// partial tile per sequence.
static int prefill_items_per_group(int num_seqs, int num_tokens, int BT) { return (num_tokens + BT - 1) / BT + num_seqs; }

hipError_t prefill_resident_workgroups(int& resident) {
    // Two workgroups per CU are resident (LDS and register budget).
    int cus = 0;
    const hipError_t e = device_cu_count(cus);
    if (e != hipSuccess) return e;
    resident = 2 * cus;
    return hipSuccess;
}

// A split call has at most `resident` pieces in all: one counter and one
// partial slot per resident workgroup, whatever the batch.
size_t prefill_counter_bytes(int resident) { return ((size_t)resident * sizeof(int) + 255) & ~(size_t)255; }

size_t prefill_workspace_bytes(int resident) {
    return resident > 0 ? prefill_counter_bytes(resident) + (size_t)resident * kPartSlotBytes : 0;
}

int prefill_group(int n_rep) { return pick_group(n_rep); }

hipError_t launch_paged_prefill(int dtype, PrefillArgs a, int num_tokens, int decode_rows_max, hipStream_t st) {
    const int G = pick_group(a.n_rep);
    const int BT = 32 * (4 / G);
    a.head_groups = a.n_rep / G;
    a.items_per_group = prefill_items_per_group(a.num_seqs, num_tokens, BT);
    a.tiles_per_group = a.items_per_group;
    a.total_work = a.tiles_per_group * a.n_kv_heads * a.head_groups;
    if (num_tokens <= 0 || a.num_seqs <= 0) return hipSuccess;
    {
        hipError_t e = prefill_resident_workgroups(a.resident);
        if (e != hipSuccess) return e;
    }
    if (a.decode_blocks > 0) {
        if (!a.skip_decode_rows || a.dec.head_groups * G != a.n_rep) return hipErrorInvalidValue;
        a.decode_blocks = (a.decode_blocks + 7) / 8 * 8;
    }
    if (a.part) {
        hipError_t e = prefill_resident_workgroups(a.resident);
        if (e != hipSuccess) return e;
        // A split needs all pieces in the resident slots at once, and a call
        // has at least ceil(num_tokens / BT) query tiles per KV head group
        // (not counting sequences of one token when the decode workers take
        // them): when those already fill the slots the call cannot split, and
        // the kernel skips its split estimate.
        const int tile_tokens = a.skip_decode_rows ? std::max(0, num_tokens - decode_rows_max) : num_tokens;
        const int64_t min_tiles = (int64_t)((tile_tokens + BT - 1) / BT) * a.n_kv_heads * a.head_groups;
        if (min_tiles >= a.resident) {
            a.part = nullptr;
            a.counters = nullptr;
        } else {
            // a split call has at most `resident` pieces
            a.total_work = a.total_work > a.resident ? a.total_work : a.resident;
        }
    }
    hipError_t e = launch_dtype<true>(dtype, G, a, st);
    if (e == hipSuccess && a.decode_blocks > 0) e = launch_paged_decode_merge(dtype, a.dec, a.num_seqs, st);
    return e;
}

hipError_t launch_dense_attention(int dtype, PrefillArgs a, hipStream_t st) {
    const int G = pick_group(a.n_rep);
    const int BT = 32 * (4 / G);
    a.head_groups = a.n_rep / G;
    a.tiles_per_group = a.num_seqs * ((a.q_len + BT - 1) / BT);
    a.total_work = a.tiles_per_group * a.n_kv_heads * a.head_groups;
    if (a.q_len <= 0 || a.num_seqs <= 0) return hipSuccess;
    return launch_dtype<false>(dtype, G, a, st);
}

}  // namespace femto
