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
//  * KV is consumed in tiles of 64 keys (4 pages).  K is stored row-major
//    [key][dim]; V is transposed on its way into LDS to [dim][key];
//  * per tile and wave: S^T(64 x 32) = K . Q^T with 16 MFMAs (Q stays in
//    registers as the B operand), online softmax with the query index equal
//    to the lane (mod 32), then O^T(128 x 32) += V^T . P^T with 16 MFMAs, P
//    taken straight from the S^T accumulators, rounded to the storage type
//    (the reference's Triton kernel rounds P the same way, line 153-155);
//  * causal tile skipping: a wave skips tiles past its largest visible key
//    and applies the mask only on tiles that cross its smallest limit;
//  * tiles of one sequence are issued heaviest (last) first, and the work
//    list is laid out so each XCD (workgroup id mod 8) gets a contiguous
//    range of KV heads, keeping a head's pages in one L2.
#include "common.h"
#include "launch.h"

namespace femto {

constexpr int kKvTile = 64;
constexpr int kKPitch = kDimHead + 8;  // elements per K row in LDS (272 B)
constexpr int kVPitch = kKvTile + 4;   // elements per V^T row in LDS (136 B)
constexpr float kEmptyMaxP = -1.0e30f;

__device__ __forceinline__ int block_incl_scan(int v, int* s_wsum, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    if (lane == 63) s_wsum[wave] = v;
    __syncthreads();
    int off = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int x = s_wsum[w];
        off += (w < wave) ? x : 0;
        total += x;
    }
    __syncthreads();
    return v + off;
}

template <typename E, int G, bool PAGED>
__global__ __launch_bounds__(256) void attention_mfma_kernel(PrefillArgs a) {
    constexpr int EB = 2;
    constexpr int BT = 32 * (4 / G);
    __shared__ __attribute__((aligned(16))) uint16_t Ks[kKvTile * kKPitch];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[kDimHead * kVPitch];
    __shared__ int s_wsum[4];
    __shared__ int s_seq, s_ltile;
    __shared__ int s_kend[4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int h2 = lane >> 5;

    // ---- work item, XCD-aware: workgroup id mod 8 selects the XCD.
    const int per_xcd = (int)gridDim.x >> 3;
    const int lin = blockIdx.x;
    const int w = (lin & 7) * per_xcd + (lin >> 3);
    if (w >= a.total_work) return;
    const int grp = w / a.tiles_per_group;
    const int tile_lin = w - grp * a.tiles_per_group;
    const int kvh = grp / a.head_groups;
    const int hg = grp - kvh * a.head_groups;

    int b, tile, q_begin, q_end, kv_len;
    if constexpr (PAGED) {
        if (tid == 0) s_seq = -1;
        int carry = 0;
        for (int base = 0; base < a.num_seqs; base += 256) {
            const int i = base + tid;
            int nt = 0;
            if (i < a.num_seqs) {
                const int ql = a.cu_seqlens[i + 1] - a.cu_seqlens[i];
                nt = ql > 0 ? (ql + BT - 1) / BT : 0;
            }
            int total;
            const int incl = block_incl_scan(nt, s_wsum, total);
            const int excl = incl - nt;
            if (i < a.num_seqs && tile_lin >= carry + excl && tile_lin < carry + incl) {
                s_seq = i;
                s_ltile = tile_lin - carry - excl;
            }
            carry += total;
            if (carry > tile_lin) break;
        }
        __syncthreads();
        b = s_seq;
        if (b < 0) return;
        q_begin = a.cu_seqlens[b];
        q_end = a.cu_seqlens[b + 1];
        kv_len = a.kv_lens[b];
        const int nt = (q_end - q_begin + BT - 1) / BT;
        tile = nt - 1 - s_ltile;  // heaviest tile of the sequence first
    } else {
        const int tpb = (a.q_len + BT - 1) / BT;
        b = tile_lin / tpb;
        tile = tile_lin - b * tpb;
        q_begin = 0;
        q_end = a.q_len;
        kv_len = a.kv_len;
    }

    const int hw = wave % G;
    const int tb = wave / G;
    const int h = kvh * a.n_rep + hg * G + hw;
    const int t = q_begin + tile * BT + tb * 32 + l32;  // this lane's query token
    const bool qvalid = t < q_end;

    // Number of keys visible to this lane's query.
    int lim;
    if constexpr (PAGED) {
        const int pos = qvalid ? a.positions[t] : kv_len;
        lim = pos + 1 < kv_len ? pos + 1 : kv_len;
        lim = lim < 0 ? 0 : lim;
    } else {
        lim = kv_len;
    }
    int kend_w = qvalid ? lim : 0;
    int kfull_w = qvalid ? lim : 0x7fffffff;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        kend_w = max(kend_w, __shfl_xor(kend_w, o, 64));
        kfull_w = min(kfull_w, __shfl_xor(kfull_w, o, 64));
    }
    if (lane == 0) s_kend[wave] = kend_w;
    __syncthreads();
    const int kend = max(max(s_kend[0], s_kend[1]), max(s_kend[2], s_kend[3]));

    // Q rows in registers: the B operand of S^T = K . Q^T.
    u32x4 qreg[8];
    {
        const char* qrow = reinterpret_cast<const char*>(a.q) +
                           ((int64_t)b * a.q_stride_batch + (int64_t)h * a.q_stride_head + (int64_t)t * a.q_stride_token) * EB;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qreg[kk] = qvalid ? ld16(qrow + (16 * kk + 8 * h2) * EB) : u32x4{0, 0, 0, 0};
    }

    // ---- KV tile staging ------------------------------------------------
    const char* kbase_p = reinterpret_cast<const char*>(a.k);
    const char* vbase_p = reinterpret_cast<const char*>(a.v);
    const int32_t* table = PAGED ? a.tables + (int64_t)b * a.table_stride : nullptr;
    const int c16 = tid & 15;
    const int r16 = tid >> 4;

    auto key_row = [&](const char* base, int key, int64_t s0, int64_t s1, int64_t s2, bool& ok) -> const char* {
        ok = key < kv_len;
        if constexpr (PAGED) {
            const int page = key >> 4;
            const int blk = (ok && page < a.num_pages_per_seq) ? table[page] : -1;
            ok = ok && blk >= 0 && (int64_t)blk < a.num_blocks;
            return base + ((int64_t)blk * s0 + (int64_t)kvh * s1 + (int64_t)(key & 15) * s2) * EB;
        } else {
            return base + ((int64_t)b * s0 + (int64_t)kvh * s1 + (int64_t)key * s2) * EB;
        }
    };

    u32x4 kreg[4], vreg[4];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bool ok;
            const char* p = key_row(kbase_p, kb + 16 * j + r16, a.k_stride0, a.k_stride1, a.k_stride2, ok);
            kreg[j] = ok ? ld16(p + 16 * c16) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bool ok;
            const char* p = key_row(vbase_p, kb + 4 * r16 + i, a.v_stride0, a.v_stride1, a.v_stride2, ok);
            vreg[i] = ok ? ld16(p + 16 * c16) : u32x4{0, 0, 0, 0};
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) st16(&Ks[(16 * j + r16) * kKPitch + 8 * c16], kreg[j]);
        // V rows 4*r16 .. 4*r16+3, dims 8*c16 .. +7  ->  V^T[dim][4 keys]
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int word = e >> 1;
            const int sh = (e & 1) * 16;
            const uint32_t v0 = (vreg[0][word] >> sh) & 0xffffu;
            const uint32_t v1 = (vreg[1][word] >> sh) & 0xffffu;
            const uint32_t v2 = (vreg[2][word] >> sh) & 0xffffu;
            const uint32_t v3 = (vreg[3][word] >> sh) & 0xffffu;
            *reinterpret_cast<u32x2*>(&Vt[(8 * c16 + e) * kVPitch + 4 * r16]) = u32x2{v0 | (v1 << 16), v2 | (v3 << 16)};
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] = f32x16{};
    float m_run = kEmptyMaxP;
    float l_run = 0.0f;
    const float scale = a.scale_log2;

    const int ntiles = (kend + kKvTile - 1) / kKvTile;
    if (ntiles > 0) load_tile(0);
    for (int it = 0; it < ntiles; ++it) {
        const int kb = it * kKvTile;
        __syncthreads();
        store_tile();
        __syncthreads();
        if (it + 1 < ntiles) load_tile(kb + kKvTile);
        if (kb >= kend_w) continue;
        const bool need_mask = kb + kKvTile > kfull_w;

        // S^T blocks: keys kb + 32*kb2 + (0..31), queries = lanes.
        f32x16 sacc[2];
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
            sacc[kb2] = f32x16{};
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const u32x4 ka = *reinterpret_cast<const u32x4*>(&Ks[(32 * kb2 + l32) * kKPitch + 16 * kk + 8 * h2]);
                sacc[kb2] = mfma32x32x16(E{}, ka, qreg[kk], sacc[kb2]);
            }
        }
        // Accumulator i of block kb2 holds key kb + 32*kb2 + 8*(i/4) + 4*h2 + i%4.
        float mx = kEmptyMaxP;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float s = sacc[kb2][i] * scale;
                if (need_mask) {
                    const int key = kb + 32 * kb2 + 8 * (i >> 2) + 4 * h2 + (i & 3);
                    s = key < lim ? s : -INFINITY;
                }
                sacc[kb2][i] = s;
                mx = fmaxf(mx, s);
            }
        }
        mx = fmaxf(mx, shfl_xor_f32(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;

        // P^T as the B operand: k-slot j of lane half h2 in step ks is key
        // kb + 16*ks + 8*(j/4) + 4*h2 + j%4.
        u32x4 pb[4];
        float psum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float pf[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pf[j] = fast_exp2(sacc[ks >> 1][8 * (ks & 1) + j] - m_new);
                psum += pf[j];
            }
            pb[ks] = pack8(E{}, pf);
        }
        l_run += psum;

#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint16_t* vrow = &Vt[(32 * dt + l32) * kVPitch + 16 * ks + 4 * h2];
                const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
                const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
                const u32x4 va = u32x4{lo[0], lo[1], hi[0], hi[1]};
                oacc[dt] = mfma32x32x16(E{}, va, pb[ks], oacc[dt]);
            }
        }
    }

    // ---- epilogue: O^T accumulator i of dim tile dt holds dim
    // 32*dt + 8*(i/4) + 4*h2 + i%4 of this lane's query.
    const float l_tot = l_run + shfl_xor_f32(l_run, 32);
    if (qvalid) {
        char* orow = reinterpret_cast<char*>(a.out) +
                     ((int64_t)b * a.out_stride_batch + (int64_t)h * a.out_stride_head + (int64_t)t * a.out_stride_token) * EB;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * dt + 8 * g + 4 * h2;
                const u32x2 v = pack4(E{}, oacc[dt][4 * g] / l_tot, oacc[dt][4 * g + 1] / l_tot,
                                      oacc[dt][4 * g + 2] / l_tot, oacc[dt][4 * g + 3] / l_tot);
                *reinterpret_cast<u32x2*>(orow + d0 * EB) = v;
            }
        }
    }
}

static int pick_group(int n_rep) { return (n_rep % 4 == 0) ? 4 : (n_rep % 2 == 0) ? 2 : 1; }

template <typename E, bool PAGED>
static hipError_t launch_g(int G, const PrefillArgs& a, hipStream_t st) {
    const int grid = ((a.total_work + 7) / 8) * 8;
    switch (G) {
        case 1: hipLaunchKernelGGL((attention_mfma_kernel<E, 1, PAGED>), dim3(grid), dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((attention_mfma_kernel<E, 2, PAGED>), dim3(grid), dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((attention_mfma_kernel<E, 4, PAGED>), dim3(grid), dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool PAGED>
static hipError_t launch_dtype(int dtype, int G, const PrefillArgs& a, hipStream_t st) {
    switch (dtype) {
        case kDtypeBF16: return launch_g<BF16, PAGED>(G, a, st);
        case kDtypeF16: return launch_g<F16, PAGED>(G, a, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_paged_prefill(int dtype, PrefillArgs a, int num_tokens, hipStream_t st) {
    const int G = pick_group(a.n_rep);
    const int BT = 32 * (4 / G);
    a.head_groups = a.n_rep / G;
    a.tiles_per_group = (num_tokens + BT - 1) / BT + a.num_seqs;
    a.total_work = a.tiles_per_group * a.n_kv_heads * a.head_groups;
    if (num_tokens <= 0 || a.num_seqs <= 0) return hipSuccess;
    return launch_dtype<true>(dtype, G, a, st);
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
