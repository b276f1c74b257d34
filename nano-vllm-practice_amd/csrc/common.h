// Device helpers shared by the gfx950 attention kernels.
//
// Wavefronts are 64 lanes.  A "row" below is a DPP row of 16 lanes; the
// decode kernel assigns one key (16 lanes x 8 head dims) per row, so its
// dot-product reduction never leaves a DPP row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace femto {

constexpr int kPage = 16;               // tokens per KV page (kKVLenPerPage)
constexpr int kDimHead = 128;           // head dim the kernels are built for
constexpr int kMaxKVLenNonSplit = 8192; // exported for API parity
constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// log2(e): softmax runs in base 2, exp(x) = exp2(x * log2(e)).
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- DPP all-reduce inside a 16-lane row -------------------------------
// row_ror:8, row_ror:4, quad_perm [2,3,0,1], quad_perm [1,0,3,2]: after the
// four steps every lane of the row holds the row total.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f32<0x128>(x);  // row_ror:8
    x += dpp_f32<0x124>(x);  // row_ror:4
    x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
    return x;
}

__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f32<0x128>(x));
    x = fmaxf(x, dpp_f32<0x124>(x));
    x = fmaxf(x, dpp_f32<0x4E>(x));
    x = fmaxf(x, dpp_f32<0xB1>(x));
    return x;
}

// Wave total / maximum, in every lane: the four row results (lanes 0, 16,
// 32, 48) combined through scalar reads.
__device__ __forceinline__ float lane_f32(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ float wave_sum_f32(float x) {
    x = row16_sum(x);
    return (lane_f32(x, 0) + lane_f32(x, 16)) + (lane_f32(x, 32) + lane_f32(x, 48));
}
__device__ __forceinline__ float wave_max_f32(float x) {
    x = row16_max(x);
    return fmaxf(fmaxf(lane_f32(x, 0), lane_f32(x, 16)), fmaxf(lane_f32(x, 32), lane_f32(x, 48)));
}

// DPP on 32-bit ints: rows (16 lanes) enabled by kRowMask; a lane whose
// source lies outside its row, or whose row is disabled, gets 0.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ int dpp_i32(int x) {
    return __builtin_amdgcn_update_dpp(0, x, kCtrl, kRowMask, 0xf, false);
}

// Wave sum, to every lane: DPP inside each 16-lane row, then the four rows.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += dpp_i32<0x128>(v);  // row_ror:8
    v += dpp_i32<0x124>(v);  // row_ror:4
    v += dpp_i32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_i32<0xB1>(v);   // quad_perm [1,0,3,2]
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

// Wave minimum / maximum, to every lane.
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, dpp_i32<0x128>(v));
    v = max(v, dpp_i32<0x124>(v));
    v = max(v, dpp_i32<0x4E>(v));
    v = max(v, dpp_i32<0xB1>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, dpp_i32<0x128>(v));
    v = min(v, dpp_i32<0x124>(v));
    v = min(v, dpp_i32<0x4E>(v));
    v = min(v, dpp_i32<0xB1>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Inclusive scan over the 64 lanes: row_shr 1, 2, 4, 8 inside each row,
// then row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then
// the total of rows 0-1 into rows 2-3 (row_bcast:31).
__device__ __forceinline__ int wave_incl_scan_i32(int x) {
    x += dpp_i32<0x111>(x);
    x += dpp_i32<0x112>(x);
    x += dpp_i32<0x114>(x);
    x += dpp_i32<0x118>(x);
    x += dpp_i32<0x142, 0xa>(x);
    x += dpp_i32<0x143, 0xc>(x);
    return x;
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) { return __shfl_xor(x, mask, kWave); }

// Row pairs through v_permlane16_swap / v_permlane32_swap (VALU, no LDS):
// a = x of the first row of each pair (rows 0 and 2 for 16; lanes 0-31 for
// 32) and b = x of the second (rows 1 and 3; lanes 32-63), in every lane of
// the pair.
__device__ __forceinline__ void pair16(float x, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float x, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// ---- element types -----------------------------------------------------
struct BF16 {
    using mfma_vec = bf16x8;
    using quad = bf16x4;
    static constexpr int kBytes = 2;
};
struct F16 {
    using mfma_vec = f16x8;
    using quad = f16x4;
    static constexpr int kBytes = 2;
};
struct F32 {
    static constexpr int kBytes = 4;
};

// 8 x 16-bit values held in a 16-byte register quad.
__device__ __forceinline__ void unpack8(BF16, u32x4 w, float f[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ void unpack8(F16, u32x4 w, float f[8]) {
    f16x8 h = __builtin_bit_cast(f16x8, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
}

// Round-to-nearest-even conversion of 8 floats to 16-bit storage.
__device__ __forceinline__ u32x4 pack8(BF16, const float f[8]) {
    bf16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (__bf16)f[i];
    return __builtin_bit_cast(u32x4, h);
}

__device__ __forceinline__ u32x4 pack8(F16, const float f[8]) {
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)f[i];
    return __builtin_bit_cast(u32x4, h);
}

__device__ __forceinline__ u32x2 pack4(BF16, float a, float b, float c, float d) {
    bf16x4 h = {(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
    return __builtin_bit_cast(u32x2, h);
}

__device__ __forceinline__ u32x2 pack4(F16, float a, float b, float c, float d) {
    f16x4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
    return __builtin_bit_cast(u32x2, h);
}

__device__ __forceinline__ f32x16 mfma32x32x16(BF16, u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32x32x16(F16, u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// acc + sum of the 8 packed 16-bit values in w (dot products with ones).
// Each word is copied to a scalar before __builtin_bit_cast: applied to a
// vector element (w[i]) directly, the cast reads element 0 for every i.
__device__ __forceinline__ float sum8(BF16, u32x4 w, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, (uint32_t)w[i]), one, acc, false);
    return acc;
}

__device__ __forceinline__ float sum8(F16, u32x4 w, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, (uint32_t)w[i]), one, acc, false);
    return acc;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// 16 bytes with the non-temporal hint, for data read once per call (KV pages
// in decode): random 4 KiB page reads of 545 MB ran at 6.35 TB/s this way
// against 5.69 TB/s with ordinary loads.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

}  // namespace femto
