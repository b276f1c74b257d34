// Fused attention prologue: per-head RMSNorm of q and k, rotary embedding
// of both, and the KV-cache write of the rotated k and of v.
//
// Reference steps (femtovllm/models/qwen/qwen3.py:230-264 decode and
// 312-366 prefill): q = q_norm(q); k = k_norm(k) (torch.nn.RMSNorm(d_head,
// eps), qwen3.py:181-183: x / sqrt(mean(x^2) + eps) * weight); q, k =
// rotary_embd(., positions) (cos[p] * x + sin[p] * concat(-x2, x1),
// QwenRotaryEmbedding.forward, qwen3.py:97-138, per-token positions); then
// the per-sequence slicing loops write k and v into the paged pools (the
// rule of kv_cache_write.hip: sequence b's tokens at positions[q_begin] + i,
// stopping at the first table column that is -1, past the table width or
// outside the pool).  Here every step runs in fp32 and each output element
// is rounded once to the storage type (the reference rounds after the norm,
// after the weight and after each RoPE product).  cos / sin are the
// caller's fp32 tables (rope_rows, head_dim); a position outside them gives
// NaN rows, where the reference's index would raise.
//
// Work: workgroup (x, b) takes tokens q_begin + 4x .. + 3 of sequence b,
// then the four tokens gridDim.x * 4 further on, until the sequence ends.
// A token has H q rows, KVH k rows and KVH v rows of head_dim = 128; a DPP
// row of 16 lanes handles one of them, lane c holding dims 8c .. 8c + 7, so
// the sum of squares is a 16-lane DPP reduction and the RoPE partner of dim
// d (d +- 64) sits in lane c +- 8 (one DPP row rotation).  Rows move in
// batches of eight per DPP row (128 per workgroup), two batches in flight:
// the first two are loaded before the position and block-table lookups
// (which take two dependent round trips), and each register buffer is
// refilled as soon as its batch is stored.  The tokens' cos / sin rows are
// staged in LDS once per workgroup.
#include "common.h"
#include "launch.h"

namespace femto {

constexpr int kProTokens = 4;  // tokens per workgroup (a multiple of 4; at most 16, which touch at most two pages)
constexpr int kProBatch = 8;    // rows per DPP row in one batch (128 rows per workgroup)

// 8 elements at p (16 bytes for 16-bit types, 32 bytes for f32) as floats.
__device__ __forceinline__ void load8(BF16, const char* p, float f[8]) { unpack8(BF16{}, ld16(p), f); }
__device__ __forceinline__ void load8(F16, const char* p, float f[8]) { unpack8(F16{}, ld16(p), f); }
__device__ __forceinline__ void load8(F32, const char* p, float f[8]) {
    const u32x4 a = ld16(p), b = ld16(p + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = __uint_as_float(a[i]);
        f[4 + i] = __uint_as_float(b[i]);
    }
}

__device__ __forceinline__ void store8(BF16, char* p, const float f[8]) { st16(p, pack8(BF16{}, f)); }
__device__ __forceinline__ void store8(F16, char* p, const float f[8]) { st16(p, pack8(F16{}, f)); }
__device__ __forceinline__ void store8(F32, char* p, const float f[8]) {
    st16(p, u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])});
    st16(p + 16, u32x4{__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7])});
}

// Source row of row slot pi of tokens t0..: q head, k head or v head.
// Plain values in, so the three-way choice stays a register select (a
// choice among the kernel argument's fields, read through the lambdas'
// captures, compiled to a load from the argument block or from scratch at
// every use).
struct RowSrc {
    uint64_t base[3];
    int64_t tok[3], head[3];
};
template <int EB>
__device__ __forceinline__ const char* row_src(const RowSrc rs, int pi, int R, int H, int KVH, int t0, int d0) {
    const int ti = pi / R;
    const int r = pi - ti * R;
    const bool isq = r < H, isk = !isq && r < H + KVH;
    const int hr = isq ? r : isk ? r - H : r - H - KVH;
    const int64_t stt = isq ? rs.tok[0] : isk ? rs.tok[1] : rs.tok[2];
    const int64_t sth = isq ? rs.head[0] : isk ? rs.head[1] : rs.head[2];
    const uint64_t base = isq ? rs.base[0] : isk ? rs.base[1] : rs.base[2];
    return reinterpret_cast<const char*>(base) + ((int64_t)(t0 + ti) * stt + (int64_t)hr * sth + d0) * EB;
}

// Raw 16-byte chunks of one row slice (two for f32: 8 floats).
template <typename E>
struct RowRaw {
    u32x4 w[E::kBytes == 4 ? 2 : 1];
};

template <typename E>
__device__ __forceinline__ void load_raw(const char* p, RowRaw<E>& r) {
    r.w[0] = ld16(p);
    if constexpr (E::kBytes == 4) r.w[1] = ld16(p + 16);
}
template <typename E>
__device__ __forceinline__ void store_raw(char* p, const RowRaw<E>& r) {
    st16(p, r.w[0]);
    if constexpr (E::kBytes == 4) st16(p + 16, r.w[1]);
}
__device__ __forceinline__ void raw_to_float(BF16, const RowRaw<BF16>& r, float f[8]) { unpack8(BF16{}, r.w[0], f); }
__device__ __forceinline__ void raw_to_float(F16, const RowRaw<F16>& r, float f[8]) { unpack8(F16{}, r.w[0], f); }
__device__ __forceinline__ void raw_to_float(F32, const RowRaw<F32>& r, float f[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = __uint_as_float(r.w[0][i]);
        f[4 + i] = __uint_as_float(r.w[1][i]);
    }
}

template <typename E>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(PrologueArgs a) {
    constexpr int EB = E::kBytes;
    __shared__ int s_stop, s_blk[2];
    __shared__ float s_rope[kProTokens][2][kDimHead];  // cos, sin rows of the workgroup's tokens
    const int b = blockIdx.y;
    int q_begin, q_end;
    if (a.cw.cu_seqlens) {
        q_begin = a.cw.cu_seqlens[b];
        q_end = a.cw.cu_seqlens[b + 1];
    } else {  // decode: one token per sequence
        q_begin = b;
        q_end = b + 1;
    }
    const RowSrc rsrc{{(uint64_t)(uintptr_t)a.q, (uint64_t)(uintptr_t)a.cw.k, (uint64_t)(uintptr_t)a.cw.v},
                      {a.q_stride_token, a.cw.k_stride_token, a.cw.v_stride_token},
                      {a.q_stride_head, a.cw.k_stride_head, a.cw.v_stride_head}};

    // One round: tokens t0 .. t0 + kProTokens - 1 of the sequence; the first
    // keeps two batches of rows in flight, later ones (a sequence longer
    // than the max_q_len that sized the grid) load one row per DPP row at a
    // time, so that rarely used path does not raise the register count
    // (one loop around a single copy of the code needed ~220 registers, two
    // waves per SIMD instead of four: 34 instead of 22.6 us per 8 x 512 chunk).
    auto round = [&](int t0, auto two_c) __attribute__((always_inline)) {
        constexpr bool kTwo = decltype(two_c)::value;
        const int t1 = min(q_end, t0 + kProTokens);
        const int ntok = t1 - t0;
        const int tid = threadIdx.x;

        const int lrow = tid >> 4;  // DPP row of the workgroup: one (token, head row) at a time
        const int c = tid & 15;     // dims 8c .. 8c + 7
        const int d0 = 8 * c;
        const int H = a.n_heads, KVH = a.cw.n_kv_heads;
        const int R = H + 2 * KVH;  // rows per token: q heads, k heads, v heads
        const int pairs = ntok * R;

        auto src_of = [&](int pi) { return row_src<EB>(rsrc, pi, R, H, KVH, t0, d0); };
        // A batch is kProBatch rows per DPP row (128 rows per workgroup).
        auto load_batch = [&](int base, auto& raw) {
            constexpr int N = sizeof(raw) / sizeof(raw[0]);
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int pi = base + lrow + 16 * k;
                if (pi < pairs) load_raw<E>(src_of(pi), raw[k]);
            }
        };

        // The first two batches of rows depend only on cu_seqlens: their loads
        // go out before anything else, so the position and block-table lookups
        // below wait while the rows are already on their way.
        RowRaw<E> ra[kProBatch], rb[kProBatch];
        if constexpr (kTwo) {
            load_batch(0, ra);
            if (pairs > 16 * kProBatch) load_batch(16 * kProBatch, rb);
        }

        // This thread's share of the tokens' cos / sin rows: tokens tid / 64 + 4i,
        // table (tid / 32) % 2, dims 4 (tid % 32) .. + 3.
        const int rt = tid >> 6, rsel = (tid >> 5) & 1, rd = 4 * (tid & 31);
        int pr[kProTokens / 4];
#pragma unroll
        for (int i = 0; i < kProTokens / 4; ++i) pr[i] = rt + 4 * i < ntok ? a.positions_rope[t0 + rt + 4 * i] : -1;

        // Destination pages of this workgroup's tokens (as kv_cache_write_kernel;
        // they touch at most two pages).
        const int p0 = a.cw.positions[q_begin];
        const int colA = p0 >= 0 ? (p0 + (t0 - q_begin)) / kPage : 0;
        const int colB = p0 >= 0 ? (p0 + (t1 - 1 - q_begin)) / kPage : 0;
        if constexpr (!kTwo) __syncthreads();  // the previous round's readers of s_stop / s_blk / s_rope are done
        if (tid == 0) s_stop = p0 < 0 ? -1 : 0x7fffffff;
        __syncthreads();
        if (p0 >= 0) {
            const int32_t* table = a.cw.tables + (int64_t)b * a.cw.table_stride;
            for (int tc = p0 / kPage + tid; tc <= colB; tc += 256) {
                const int blk = tc < a.cw.num_pages_per_seq ? table[tc] : -1;
                if (blk < 0 || (int64_t)blk >= a.cw.num_blocks) atomicMin(&s_stop, tc);
                if (tc == colA) s_blk[0] = blk;
                if (tc == colB) s_blk[1] = blk;
            }
        }
#pragma unroll
        for (int i = 0; i < kProTokens / 4; ++i) {
            float4 v4;
            if (pr[i] >= 0 && pr[i] < a.rope_rows) {
                const float* tab = rsel ? a.sin : a.cos;
                v4 = *reinterpret_cast<const float4*>(tab + (int64_t)pr[i] * a.rope_stride + rd);
            } else {  // a position outside the tables: NaN rows
                v4 = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
            }
            if (rt + 4 * i < ntok) *reinterpret_cast<float4*>(&s_rope[rt + 4 * i][rsel][rd]) = v4;
        }
        float wq[8], wk[8];
        load8(E{}, static_cast<const char*>(a.q_weight) + d0 * EB, wq);
        load8(E{}, static_cast<const char*>(a.k_weight) + d0 * EB, wk);
        __syncthreads();
        const int stop = s_stop;

        // Norm, rotate and store one batch.
        auto process = [&](int base, const auto& raw) {
            constexpr int N = sizeof(raw) / sizeof(raw[0]);
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int pi = base + lrow + 16 * k;  // uniform within the DPP row
                if (pi >= pairs) break;
                const int ti = pi / R;
                const int r = pi - ti * R;
                const int t = t0 + ti;
                const int pc = p0 + (t - q_begin);  // cache position
                const int col = pc / kPage;
                const bool write_cache = p0 >= 0 && col < stop;
                char* dst = nullptr;
                if (r >= H && write_cache) {
                    const int h = r < H + KVH ? r - H : r - H - KVH;
                    const int blk = s_blk[col == colA ? 0 : 1];
                    const int64_t el = (int64_t)blk * a.cw.pool_stride_block + (int64_t)h * a.cw.pool_stride_head +
                                       (int64_t)(pc % kPage) * a.cw.pool_stride_row + d0;
                    dst = static_cast<char*>(r < H + KVH ? a.cw.k_pool : a.cw.v_pool) + el * EB;
                }
                if (r >= H + KVH) {  // v: plain copy
                    if (dst) store_raw<E>(dst, raw[k]);
                    continue;
                }
                const bool is_q = r < H;
                float x[8];
                raw_to_float(E{}, raw[k], x);
                // RMSNorm over the 128 dims of the row.
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
                ss = row16_sum(ss);
                const float rinv = 1.0f / sqrtf(ss * (1.0f / kDimHead) + a.eps);
                const float* w = is_q ? wq : wk;
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = x[i] * rinv * w[i];
                // RoPE at this token's position: rot(x)[d] = -x[d + 64] for d < 64, x[d - 64] above.
                float o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float partner = dpp_f32<0x128>(x[i]);  // lane c +- 8 (row_ror:8)
                    const float rot = c < 8 ? -partner : partner;
                    o[i] = fmaf(s_rope[ti][0][d0 + i], x[i], s_rope[ti][1][d0 + i] * rot);
                }
                if (is_q) {
                    char* qo = static_cast<char*>(a.q_out) +
                               ((int64_t)t * a.q_out_stride_token + (int64_t)r * a.q_out_stride_head + d0) * EB;
                    store8(E{}, qo, o);
                } else if (dst) {
                    store8(E{}, dst, o);
                }
            }
        };

        // Two batches in flight: each buffer is refilled as soon as its batch is stored.
        constexpr int kB = 16 * kProBatch;
        if constexpr (kTwo) {
            for (int base = 0; base < pairs; base += 2 * kB) {
                process(base, ra);
                if (base + 2 * kB < pairs) load_batch(base + 2 * kB, ra);
                if (base + kB < pairs) {
                    process(base + kB, rb);
                    if (base + 3 * kB < pairs) load_batch(base + 3 * kB, rb);
                }
            }
        } else {
            RowRaw<E> r1[1];
            for (int base = 0; base < pairs; base += 16) {
                load_batch(base, r1);
                process(base, r1);
            }
        }
    };
    // max_q_len only sizes the grid: a sequence longer than it is covered by
    // later rounds of the same workgroups (the loop condition is uniform
    // across the workgroup, so the barriers inside stay matched).
    const int first = q_begin + (int)blockIdx.x * kProTokens;
    if (first >= q_end) return;
    round(first, std::true_type{});
    for (int t0 = first + (int)gridDim.x * kProTokens; t0 < q_end; t0 += (int)gridDim.x * kProTokens)
        round(t0, std::false_type{});
}

hipError_t launch_qk_norm_rope(int dtype, const PrologueArgs& a, int max_q_len, hipStream_t st) {
    if (a.cw.num_seqs <= 0 || max_q_len <= 0) return hipSuccess;
    const dim3 grid((max_q_len + kProTokens - 1) / kProTokens, a.cw.num_seqs);
    switch (dtype) {
        case kDtypeBF16: hipLaunchKernelGGL(qk_norm_rope_kernel<BF16>, grid, dim3(256), 0, st, a); break;
        case kDtypeF16: hipLaunchKernelGGL(qk_norm_rope_kernel<F16>, grid, dim3(256), 0, st, a); break;
        case kDtypeF32: hipLaunchKernelGGL(qk_norm_rope_kernel<F32>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace femto
