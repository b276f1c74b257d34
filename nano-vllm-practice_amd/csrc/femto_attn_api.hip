// C ABI of libfemto_attn.so: argument checks, launch planning, dispatch.
//
// The checks mirror the reference host wrappers
// (csrc/paged_attention/paged_attention_gemv.cu:231-274,
// csrc/paged_attention/paged_attention_gemm.cu:314-353,
// csrc/flash_attention/flash_attention_warp.cu:306-349) for what can be seen
// from raw pointers and sizes; tensor-level checks (device, rank, int32
// index dtype) live in the Python layer that owns the tensors.
#include <algorithm>
#include <cmath>
#include <atomic>
#include <mutex>
#include <string>

#include "common.h"
#include "femto_attn.h"
#include "launch.h"

// Scratch of femto_paged_attention_gemv_noalloc (see scratch_pointer below).
constexpr size_t kScratchBytes = (size_t)64 << 20;  // 64 MiB per GPU
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local std::string g_err;

// Decode calls whose max_kv_len is at most this run as one launch (a
// workgroup per sequence and KV head group, no workspace); longer ones use
// the split workers and the merge kernel.
std::atomic<int> g_single_max_kv{1024};

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return FEMTO_OK;
    return fail(FEMTO_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

const char* dtype_name(int dtype) {
    switch (dtype) {
        case FEMTO_F32: return "Float";
        case FEMTO_F16: return "Half";
        case FEMTO_BF16: return "BFloat16";
        default: return "unknown";
    }
}

int elem_bytes(int dtype) { return dtype == FEMTO_F32 ? 4 : 2; }

float scale_log2(int head_dim) { return femto::kLog2e / std::sqrt((float)head_dim); }

int check_paged_common(const char* fn, int dtype, const void* q, const void* out, const void* k_pool,
                              const void* v_pool, int64_t num_blocks, int n_kv_heads, int block_size,
                              int head_dim, int64_t ps0, int64_t ps1, int64_t ps2, int n_heads,
                              int64_t q_s0, int64_t q_s1, const int32_t* tables, int num_pages_per_seq,
                              int64_t table_stride, bool decode) {
    std::string f(fn);
    // head_dim <= 128 as the reference checks (decode:
    // paged_attention_gemv.cu:256-257; prefill: paged_attention_gemm.cu:347-348),
    // in whole 16-byte chunks for decode (a lane loads 16-byte pieces of a
    // row) and in multiples of 16 for prefill (one score MFMA step).
    const int unit = decode ? 16 / elem_bytes(dtype) : 16;
    if (head_dim <= 0 || head_dim > femto::kDimHead || head_dim % unit != 0)
        return fail(FEMTO_ERR_UNSUPPORTED,
                    f + ": head_dim must be at most " + std::to_string(femto::kDimHead) + " and a multiple of " +
                        (decode ? "16 bytes (" + std::to_string(unit) + " elements)" : std::string("16")) +
                        ", got " + std::to_string(head_dim));
    if (block_size != femto::kPage)
        return fail(FEMTO_ERR_INVALID, f + ": block_size must be " + std::to_string(femto::kPage) + ", got " +
                                           std::to_string(block_size));
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0)
        return fail(FEMTO_ERR_INVALID, f + ": n_heads (" + std::to_string(n_heads) +
                                           ") must be a positive multiple of n_kv_heads (" +
                                           std::to_string(n_kv_heads) + ")");
    if (num_blocks < 1 || num_pages_per_seq < 0 || table_stride < 0)
        return fail(FEMTO_ERR_INVALID, f + ": the pool needs at least one block and table sizes must be >= 0");
    if (!q || !out || !k_pool || !v_pool || (num_pages_per_seq > 0 && !tables))
        return fail(FEMTO_ERR_INVALID, f + ": null pointer argument");
    const int vec = 16 / elem_bytes(dtype);
    if (!aligned(q, 16) || !aligned(k_pool, 16) || !aligned(v_pool, 16) || !aligned(out, 8))
        return fail(FEMTO_ERR_INVALID, f + ": q, k_pool and v_pool must be 16-byte aligned, out 8-byte aligned");
    if (ps0 % vec || ps1 % vec || ps2 % vec || q_s0 % vec || q_s1 % vec)
        return fail(FEMTO_ERR_INVALID, f + ": pool and q strides must be multiples of 16 bytes");
    return FEMTO_OK;
}

// ---- scratch of the allocation-free decode entry point ----------------------
// femto_paged_attention_gemv_noalloc keeps its partial softmax states here
// instead of a caller workspace: a file-scope device array, one copy per GPU
// the library runs on, held until the process ends.  Host code never uses the
// array's name as an address (on the host it names a stand-in, not device
// memory); the device address comes from hipGetSymbolAddress, once per device
// on the entry point's first call there, and only that pointer reaches the
// kernels.  Every call on one GPU shares the array (it keeps the last call's
// contents; decode needs no zero-filled state), so calls that may overlap on
// one GPU (other streams, other threads) race.
// (The array itself is declared at file scope above this namespace.)
// Largest num_seqs * n_heads that still fits two partial slots per (sequence,
// head): (64 MiB) / (2 * 130 floats) ~ 64.5 k, e.g. 2048 sequences x 32 heads.
constexpr int64_t kScratchMaxSeqHeads = (int64_t)(kScratchBytes / (2 * (femto::kDimHead + 2) * sizeof(float)));

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up on first use.
int scratch_pointer(const std::string& fn, void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, (fn + ": hipGetDevice").c_str());
    if (dev < 0 || dev >= kMaxDevices) return fail(FEMTO_ERR_UNSUPPORTED, fn + ": device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, (fn + ": hipGetSymbolAddress(scratch)").c_str());
        if (!p) return fail(FEMTO_ERR_HIP, fn + ": hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return FEMTO_OK;
}

std::atomic<int> g_cu_count[kMaxDevices] = {};

}  // namespace

namespace femto {

hipError_t device_cu_count(int& cus) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        if (n <= 0) n = 1;
        g_cu_count[dev].store(n, std::memory_order_relaxed);  // every thread stores the same value
    }
    cus = n;
    return hipSuccess;
}

DecodePlan plan_paged_decode(int n_heads, int n_kv_heads, int max_kv_len, int dtype) {
    DecodePlan p;
    const int n_rep = (n_kv_heads > 0) ? n_heads / n_kv_heads : 1;
    // f32 pages take twice the registers: at most 4 query heads per wave
    p.nrep_tile = (n_rep % 8 == 0 && dtype != kDtypeF32) ? 8 : (n_rep % 4 == 0) ? 4 : (n_rep % 2 == 0) ? 2 : 1;
    const int max_pages = max_kv_len > 0 ? (max_kv_len + kPage - 1) / kPage : 1;
    // A wave's slice is at least min_chunk_pages long, so a sequence is cut
    // into at most max_slots - 1 slices (+1 for a slice straddling its start).
    p.min_chunk_pages = std::max(4, (max_pages + 31) / 32);
    p.min_chunk_pages = std::max(p.min_chunk_pages, (max_pages + 126) / 127);  // merge kernel: <= 128 slots
    p.max_slots = (max_pages + p.min_chunk_pages - 1) / p.min_chunk_pages + 1;
    return p;
}

size_t decode_workspace_bytes(int num_seqs, int n_heads, int max_slots) {
    if (num_seqs <= 0) return 0;
    const size_t slots = (size_t)num_seqs * n_heads * max_slots;
    size_t bytes = slots * (kDimHead + 2) * sizeof(float);
    return bytes + (size_t)num_seqs * sizeof(int);
}

// Kernel arguments of a decode launch over the pools; q rows / out rows b
// (decode call) or cu_seqlens[b] (decode rows of a prefill call).
DecodeArgs decode_args(const DecodePlan& plan, const void* q, int64_t q_stride_head, int64_t q_stride_row, void* out,
                       int64_t out_stride_head, int64_t out_stride_row, const void* k_pool, const void* v_pool,
                       int64_t num_blocks, int n_kv_heads, int head_dim, int64_t pool_stride_block,
                       int64_t pool_stride_head, int64_t pool_stride_row, const int32_t* kv_page_tables,
                       int num_pages_per_seq, int64_t table_stride, const int32_t* kv_lens, int num_seqs, int n_heads,
                       void* workspace) {
    DecodeArgs a{};
    a.q = q;
    a.q_stride_head = q_stride_head;
    a.q_stride_seq = q_stride_row;
    a.out = out;
    a.out_stride_head = out_stride_head;
    a.out_stride_seq = out_stride_row;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.num_blocks = num_blocks;
    a.pool_stride_block = pool_stride_block;
    a.pool_stride_head = pool_stride_head;
    a.pool_stride_row = pool_stride_row;
    a.tables = kv_page_tables;
    a.table_stride = table_stride;
    a.num_pages_per_seq = num_pages_per_seq;
    a.kv_lens = kv_lens;
    a.n_heads = n_heads;
    a.n_rep = n_heads / n_kv_heads;
    a.head_groups = a.n_rep / plan.nrep_tile;
    a.num_seqs = num_seqs;
    a.grid_heads = n_heads / plan.nrep_tile;
    a.min_chunk_pages = plan.min_chunk_pages;
    a.max_slots = plan.max_slots;
    a.head_dim = head_dim;
    a.scale_log2 = ::scale_log2(head_dim);
    const size_t slots = (size_t)num_seqs * n_heads * plan.max_slots;
    a.part_acc = static_cast<float*>(workspace);
    a.part_ml = a.part_acc + slots * kDimHead;
    a.seq_slots = reinterpret_cast<int*>(a.part_ml + slots * 2);
    return a;
}

// Upper bound on the sequences of exactly one query token in a varlen call of
// num_seqs sequences, num_tokens tokens and at most max_q_len tokens each:
// with d such sequences, num_tokens <= d + (num_seqs - d) * max_q_len.  Zero
// proves there are none (e.g. every chunked prefill call of full chunks), and
// then no decode launch is made.  The bound only decides whether to launch:
// when it is positive the decode kernel takes every one-token sequence, and
// when a max_q_len below the longest chunk makes it zero the prefill kernel
// keeps every row itself, so either way each row is computed once.
int decode_rows_bound(int num_seqs, int num_tokens, int max_q_len) {
    if (max_q_len <= 1) return num_seqs;
    const int64_t d = ((int64_t)num_seqs * max_q_len - num_tokens) / (max_q_len - 1);
    return (int)std::max<int64_t>(0, std::min<int64_t>(num_seqs, d));
}

}  // namespace femto

// Decode entry points: femto_paged_attention_gemv (workspace from the caller)
// and femto_paged_attention_gemv_noalloc (workspace = this device's scratch).
static int paged_decode_entry(const char* fn_name, int dtype, const void* q, int64_t q_stride_head,
                              int64_t q_stride_seq, void* out, int64_t out_stride_head, int64_t out_stride_seq,
                              const void* k_pool, const void* v_pool, int64_t num_blocks, int n_kv_heads,
                              int block_size, int head_dim, int64_t pool_stride_block, int64_t pool_stride_head,
                              int64_t pool_stride_row, const int32_t* kv_page_tables, int num_pages_per_seq,
                              int64_t table_stride, const int32_t* kv_lens, int num_seqs, int n_heads, int max_kv_len,
                              bool use_scratch, void* workspace, size_t workspace_bytes, void* stream) {
    g_err.clear();
    const std::string fn(fn_name);
    if (dtype != FEMTO_F32 && dtype != FEMTO_F16 && dtype != FEMTO_BF16)
        return fail(FEMTO_ERR_UNSUPPORTED, fn + ": dtype " + dtype_name(dtype) + " is not supported");
    if (num_seqs < 0 || max_kv_len < 0) return fail(FEMTO_ERR_INVALID, fn + ": negative size");
    if (num_seqs == 0) return FEMTO_OK;
    if (!kv_lens) return fail(FEMTO_ERR_INVALID, fn + ": null kv_lens");
    int rc = check_paged_common(fn_name, dtype, q, out, k_pool, v_pool, num_blocks, n_kv_heads,
                                block_size, head_dim, pool_stride_block, pool_stride_head, pool_stride_row, n_heads,
                                q_stride_head, q_stride_seq, kv_page_tables, num_pages_per_seq, table_stride, true);
    if (rc != FEMTO_OK) return rc;

    femto::DecodePlan plan = femto::plan_paged_decode(n_heads, n_kv_heads, max_kv_len, dtype);
    if (max_kv_len <= g_single_max_kv.load(std::memory_order_relaxed)) {
        // One launch, no workspace.  A max_kv_len below the true longest
        // context only makes the call slower (each wave walks its share of
        // the sequence, whatever the length).  With at most 256 (sequence,
        // query head) pairs the workgroups do not fill the GPU: one query
        // head per wave and eight waves per workgroup halve each wave's pages.
        const bool wide = (int64_t)num_seqs * n_heads <= 256;
        if (wide) plan.nrep_tile = 1;
        femto::DecodeArgs a = femto::decode_args(
            plan, q, q_stride_head, q_stride_seq, out, out_stride_head, out_stride_seq, k_pool, v_pool, num_blocks,
            n_kv_heads, head_dim, pool_stride_block, pool_stride_head, pool_stride_row, kv_page_tables,
            num_pages_per_seq, table_stride, kv_lens, num_seqs, n_heads, nullptr);
        a.single_waves = wide ? 8 : 4;
        return hip_status(femto::launch_paged_decode(dtype, a, plan.nrep_tile, num_seqs, true,
                                                     static_cast<hipStream_t>(stream)),
                          (fn + " launch").c_str());
    }
    if (use_scratch) {
        // The partial slots must fit the scratch array: with fewer slots per
        // (sequence, head) a sequence is cut into fewer, longer slices (the
        // kernel sizes slices from the longest sequence and max_slots).
        const size_t per_slot = (size_t)num_seqs * n_heads * (femto::kDimHead + 2) * sizeof(float);
        const size_t fixed = (size_t)num_seqs * sizeof(int);
        const size_t fit = kScratchBytes > fixed ? (kScratchBytes - fixed) / per_slot : 0;
        if (fit < 2)
            return fail(FEMTO_ERR_INVALID,
                        fn + ": num_seqs * n_heads = " + std::to_string((int64_t)num_seqs * n_heads) +
                            " exceeds the scratch limit of " + std::to_string(kScratchMaxSeqHeads) +
                            " (sequences x query heads); use femto_paged_attention_gemv with a workspace");
        if ((size_t)plan.max_slots > fit) {
            const int max_pages = max_kv_len > 0 ? (max_kv_len + femto::kPage - 1) / femto::kPage : 1;
            plan.max_slots = (int)fit;
            plan.min_chunk_pages = std::max(plan.min_chunk_pages, (max_pages + plan.max_slots - 2) / (plan.max_slots - 1));
        }
        rc = scratch_pointer(fn, &workspace);
        if (rc != FEMTO_OK) return rc;
        workspace_bytes = kScratchBytes;
    }
    const size_t need = femto::decode_workspace_bytes(num_seqs, n_heads, plan.max_slots);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(FEMTO_ERR_INVALID, fn + ": workspace of " + std::to_string(need) +
                                           " bytes (256-byte aligned) required, got " +
                                           std::to_string(workspace_bytes));

    const femto::DecodeArgs a = femto::decode_args(
        plan, q, q_stride_head, q_stride_seq, out, out_stride_head, out_stride_seq, k_pool, v_pool, num_blocks,
        n_kv_heads, head_dim, pool_stride_block, pool_stride_head, pool_stride_row, kv_page_tables, num_pages_per_seq,
        table_stride, kv_lens, num_seqs, n_heads, workspace);
    return hip_status(femto::launch_paged_decode(dtype, a, plan.nrep_tile, num_seqs, false,
                                                 static_cast<hipStream_t>(stream)),
                      (fn + " launch").c_str());
}

// Decode-row part of a prefill call's workspace (after the key-split part):
// the decode kernel's partial slots for every sequence, sized for the table
// width, when the call may hold sequences of one query token.
static femto::DecodePlan gemm_decode_plan(int n_heads, int n_kv_heads, int num_pages_per_seq) {
    const int64_t max_kv = std::min<int64_t>((int64_t)num_pages_per_seq * femto::kPage, 1 << 30);
    return femto::plan_paged_decode(n_heads, n_kv_heads, (int)std::max<int64_t>(1, max_kv), femto::kDtypeBF16);
}
static size_t gemm_decode_bytes(int num_seqs, int num_tokens, int max_q_len, int n_heads, int n_kv_heads,
                                int num_pages_per_seq) {
    if (femto::decode_rows_bound(num_seqs, num_tokens, max_q_len) == 0) return 0;
    const femto::DecodePlan plan = gemm_decode_plan(n_heads, n_kv_heads, num_pages_per_seq);
    return (femto::decode_workspace_bytes(num_seqs, n_heads, plan.max_slots) + 255) & ~(size_t)255;
}

extern "C" {

const char* femto_attn_last_error(void) { return g_err.c_str(); }

int femto_attn_max_kv_len_non_split(void) { return femto::kMaxKVLenNonSplit; }
int femto_attn_kv_len_per_page(void) { return femto::kPage; }
int femto_attn_dim_head(void) { return femto::kDimHead; }

int femto_attn_set_decode_single_max_kv(int max_kv_len) {
    return g_single_max_kv.exchange(max_kv_len < -1 ? -1 : max_kv_len, std::memory_order_relaxed);
}

size_t femto_paged_attention_gemm_workspace_size(int num_seqs, int num_tokens, int max_q_len, int n_heads,
                                                 int n_kv_heads, int num_pages_per_seq) {
    if (num_seqs <= 0 || num_tokens <= 0 || n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads) return 0;
    int resident = 0;
    if (femto::prefill_resident_workgroups(resident) != hipSuccess) return 0;
    return femto::prefill_workspace_bytes(resident) +
           gemm_decode_bytes(num_seqs, num_tokens, max_q_len, n_heads, n_kv_heads, num_pages_per_seq);
}

size_t femto_paged_attention_gemm_split_bytes(void) {
    int resident = 0;
    if (femto::prefill_resident_workgroups(resident) != hipSuccess) return 0;
    return femto::prefill_counter_bytes(resident);
}

size_t femto_paged_attention_gemv_workspace_size(int num_seqs, int n_heads, int max_kv_len) {
    if (num_seqs <= 0 || n_heads <= 0) return 0;
    const femto::DecodePlan p = femto::plan_paged_decode(n_heads, 1, max_kv_len, femto::kDtypeBF16);  // slots only
    return femto::decode_workspace_bytes(num_seqs, n_heads, p.max_slots);
}


int femto_paged_attention_gemv(int dtype, const void* q, int64_t q_stride_head, int64_t q_stride_seq, void* out,
                               int64_t out_stride_head, int64_t out_stride_seq, const void* k_pool,
                               const void* v_pool, int64_t num_blocks, int n_kv_heads, int block_size,
                               int head_dim, int64_t pool_stride_block, int64_t pool_stride_head,
                               int64_t pool_stride_row, const int32_t* kv_page_tables, int num_pages_per_seq,
                               int64_t table_stride, const int32_t* kv_lens, int num_seqs, int n_heads,
                               int max_kv_len, void* workspace, size_t workspace_bytes, void* stream) {
    return paged_decode_entry("paged_attention_gemv", dtype, q, q_stride_head, q_stride_seq, out, out_stride_head,
                              out_stride_seq, k_pool, v_pool, num_blocks, n_kv_heads, block_size, head_dim,
                              pool_stride_block, pool_stride_head, pool_stride_row, kv_page_tables,
                              num_pages_per_seq, table_stride, kv_lens, num_seqs, n_heads, max_kv_len, false,
                              workspace, workspace_bytes, stream);
}

int femto_paged_attention_gemv_noalloc(int dtype, const void* q, int64_t q_stride_head, int64_t q_stride_seq,
                                       void* out, int64_t out_stride_head, int64_t out_stride_seq,
                                       const void* k_pool, const void* v_pool, int64_t num_blocks, int n_kv_heads,
                                       int block_size, int head_dim, int64_t pool_stride_block,
                                       int64_t pool_stride_head, int64_t pool_stride_row,
                                       const int32_t* kv_page_tables, int num_pages_per_seq, int64_t table_stride,
                                       const int32_t* kv_lens, int num_seqs, int n_heads, int max_kv_len,
                                       void* stream) {
    return paged_decode_entry("paged_attention_gemv_noalloc", dtype, q, q_stride_head, q_stride_seq, out,
                              out_stride_head, out_stride_seq, k_pool, v_pool, num_blocks, n_kv_heads, block_size,
                              head_dim, pool_stride_block, pool_stride_head, pool_stride_row, kv_page_tables,
                              num_pages_per_seq, table_stride, kv_lens, num_seqs, n_heads, max_kv_len, true, nullptr,
                              0, stream);
}

int femto_paged_attention_gemm(int dtype, const void* q, int64_t q_stride_head, int64_t q_stride_token, void* out,
                               int64_t out_stride_head, int64_t out_stride_token, const void* k_pool,
                               const void* v_pool, int64_t num_blocks, int n_kv_heads, int block_size,
                               int head_dim, int64_t pool_stride_block, int64_t pool_stride_head,
                               int64_t pool_stride_row, const int32_t* cu_seqlens, int num_seqs, int num_tokens,
                               int max_q_len, int n_heads, const int32_t* kv_page_tables, int num_pages_per_seq,
                               int64_t table_stride, const int32_t* kv_lens, const int32_t* positions,
                               void* workspace, size_t workspace_bytes, void* stream) {
    g_err.clear();
    if (dtype != FEMTO_F16 && dtype != FEMTO_BF16)
        return fail(FEMTO_ERR_UNSUPPORTED, std::string("paged_attention_gemm: not implemented for '") +
                                               dtype_name(dtype) + "' (bf16 / f16 MFMA only)");
    if (num_seqs < 0 || num_tokens < 0 || max_q_len < 0)
        return fail(FEMTO_ERR_INVALID, "paged_attention_gemm: negative size");
    if (num_seqs == 0 || num_tokens == 0) return FEMTO_OK;
    if (!cu_seqlens || !kv_lens || !positions)
        return fail(FEMTO_ERR_INVALID, "paged_attention_gemm: null cu_seqlens / kv_lens / positions");
    int rc = check_paged_common("paged_attention_gemm", dtype, q, out, k_pool, v_pool, num_blocks, n_kv_heads,
                                block_size, head_dim, pool_stride_block, pool_stride_head, pool_stride_row, n_heads,
                                q_stride_head, q_stride_token, kv_page_tables, num_pages_per_seq, table_stride, false);
    if (rc != FEMTO_OK) return rc;
    if (out_stride_head % 4 || out_stride_token % 4)
        return fail(FEMTO_ERR_INVALID, "paged_attention_gemm: out strides must be multiples of 8 bytes");
    if (pool_stride_row < 0 || pool_stride_row > (1 << 24))
        return fail(FEMTO_ERR_INVALID, "paged_attention_gemm: pool row stride out of range");

    femto::PrefillArgs a{};
    a.q = q;
    a.q_stride_batch = 0;
    a.q_stride_head = q_stride_head;
    a.q_stride_token = q_stride_token;
    a.out = out;
    a.out_stride_batch = 0;
    a.out_stride_head = out_stride_head;
    a.out_stride_token = out_stride_token;
    a.k = k_pool;
    a.v = v_pool;
    a.k_stride0 = a.v_stride0 = pool_stride_block;
    a.k_stride1 = a.v_stride1 = pool_stride_head;
    a.k_stride2 = a.v_stride2 = pool_stride_row;
    a.num_blocks = num_blocks;
    a.cu_seqlens = cu_seqlens;
    a.tables = kv_page_tables;
    a.table_stride = table_stride;
    a.num_pages_per_seq = num_pages_per_seq;
    a.kv_lens = kv_lens;
    a.positions = positions;
    a.num_seqs = num_seqs;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.n_rep = n_heads / n_kv_heads;
    a.head_dim = head_dim;
    a.scale_log2 = scale_log2(head_dim);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int decode_rows = 0;
    if (workspace) {
        int resident = 0;
        rc = hip_status(femto::prefill_resident_workgroups(resident), "paged_attention_gemm: device query");
        if (rc != FEMTO_OK) return rc;
        const size_t split_bytes = femto::prefill_workspace_bytes(resident);
        const size_t need = split_bytes + gemm_decode_bytes(num_seqs, num_tokens, max_q_len, n_heads, n_kv_heads,
                                                            num_pages_per_seq);
        if (workspace_bytes < need || !aligned(workspace, 256))
            return fail(FEMTO_ERR_INVALID, "paged_attention_gemm: workspace of " + std::to_string(need) +
                                               " bytes (256-byte aligned) required, got " +
                                               std::to_string(workspace_bytes));
        a.counters = static_cast<int*>(workspace);
        a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + femto::prefill_counter_bytes(resident));
        if (need > split_bytes) {
            // Sequences of one query token (decode rows of a mixed batch) run
            // on the decode kernel's wave workers, which stream their pages at
            // HBM speed (an MFMA tile would hold one valid row of 32).  When
            // the workers take as many query heads per wave as a tile takes
            // (every head ratio but multiples of 8) they run in the same
            // launch as the tiles, which fill the CU slots beside them; else
            // the decode kernel runs first.
            const femto::DecodePlan plan = gemm_decode_plan(n_heads, n_kv_heads, num_pages_per_seq);
            femto::DecodeArgs d = femto::decode_args(
                plan, q, q_stride_head, q_stride_token, out, out_stride_head, out_stride_token, k_pool, v_pool,
                num_blocks, n_kv_heads, head_dim, pool_stride_block, pool_stride_head, pool_stride_row,
                kv_page_tables, num_pages_per_seq, table_stride, kv_lens, num_seqs, n_heads,
                static_cast<char*>(workspace) + split_bytes);
            d.cu_seqlens = cu_seqlens;
            d.positions = positions;
            a.skip_decode_rows = 1;
            decode_rows = femto::decode_rows_bound(num_seqs, num_tokens, max_q_len);
            if (plan.nrep_tile == femto::prefill_group(a.n_rep)) {
                a.decode_blocks = femto::decode_worker_blocks(d);
                if (a.decode_blocks <= 0) return fail(FEMTO_ERR_HIP, "paged_attention_gemm: device query");
                a.dec = d;
            } else {
                rc = hip_status(femto::launch_paged_decode(dtype, d, plan.nrep_tile, num_seqs, false, st),
                                "paged_attention_gemm decode-row launch");
                if (rc != FEMTO_OK) return rc;
            }
        }
    }
    return hip_status(femto::launch_paged_prefill(dtype, a, num_tokens, decode_rows, st), "paged_attention_gemm launch");
}

int femto_kv_cache_write(int dtype, const void* k, int64_t k_stride_token, int64_t k_stride_head, const void* v,
                         int64_t v_stride_token, int64_t v_stride_head, void* k_pool, void* v_pool,
                         int64_t num_blocks, int n_kv_heads, int block_size, int head_dim,
                         int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
                         const int32_t* cu_seqlens, int num_seqs, int num_tokens, int max_q_len,
                         const int32_t* positions, const int32_t* kv_page_tables, int num_pages_per_seq,
                         int64_t table_stride, void* stream) {
    g_err.clear();
    const std::string f = "kv_cache_write";
    if (dtype != FEMTO_F32 && dtype != FEMTO_F16 && dtype != FEMTO_BF16)
        return fail(FEMTO_ERR_UNSUPPORTED, f + ": unsupported dtype " + std::to_string(dtype));
    if (num_seqs < 0 || num_tokens < 0 || max_q_len < 0) return fail(FEMTO_ERR_INVALID, f + ": negative size");
    if (num_seqs == 0 || num_tokens == 0) return FEMTO_OK;
    if (!cu_seqlens && num_tokens != num_seqs)
        return fail(FEMTO_ERR_INVALID, f + ": without cu_seqlens every sequence has one token (num_tokens == num_seqs)");
    if (!cu_seqlens && max_q_len < 1) return fail(FEMTO_ERR_INVALID, f + ": max_q_len must be >= 1");
    if (num_seqs > 65535) return fail(FEMTO_ERR_INVALID, f + ": at most 65535 sequences per call");
    if (block_size != femto::kPage)
        return fail(FEMTO_ERR_INVALID, f + ": block_size must be " + std::to_string(femto::kPage) + ", got " +
                                           std::to_string(block_size));
    const int eb = elem_bytes(dtype);
    if (n_kv_heads <= 0 || head_dim <= 0 || (head_dim * eb) % 16 != 0)
        return fail(FEMTO_ERR_INVALID, f + ": head_dim * element size must be a positive multiple of 16 bytes");
    if (num_blocks < 1) return fail(FEMTO_ERR_INVALID, f + ": the pool needs at least one block");
    if (!k || !v || !k_pool || !v_pool || !positions || !kv_page_tables)
        return fail(FEMTO_ERR_INVALID, f + ": null pointer argument");
    if (num_pages_per_seq < 0 || table_stride < num_pages_per_seq)
        return fail(FEMTO_ERR_INVALID, f + ": table stride smaller than its width");
    if (!aligned(k, 16) || !aligned(v, 16) || !aligned(k_pool, 16) || !aligned(v_pool, 16))
        return fail(FEMTO_ERR_INVALID, f + ": k, v and the pools must be 16-byte aligned");
    const int64_t step = 16 / eb;  // elements per 16 bytes
    if (k_stride_token % step || k_stride_head % step || v_stride_token % step || v_stride_head % step ||
        pool_stride_block % step || pool_stride_head % step || pool_stride_row % step)
        return fail(FEMTO_ERR_INVALID, f + ": strides must be multiples of 16 bytes");

    femto::CacheWriteArgs a{};
    a.k = k;
    a.v = v;
    a.k_stride_token = k_stride_token;
    a.k_stride_head = k_stride_head;
    a.v_stride_token = v_stride_token;
    a.v_stride_head = v_stride_head;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.num_blocks = num_blocks;
    a.pool_stride_block = pool_stride_block;
    a.pool_stride_head = pool_stride_head;
    a.pool_stride_row = pool_stride_row;
    a.cu_seqlens = cu_seqlens;
    a.positions = positions;
    a.tables = kv_page_tables;
    a.table_stride = table_stride;
    a.num_pages_per_seq = num_pages_per_seq;
    a.num_seqs = num_seqs;
    a.n_kv_heads = n_kv_heads;
    a.row_chunks = head_dim * eb / 16;
    a.elem_bytes = eb;
    return hip_status(femto::launch_kv_cache_write(a, cu_seqlens ? max_q_len : 1, static_cast<hipStream_t>(stream)),
                      "kv_cache_write launch");
}

int femto_qk_norm_rope_cache_write(int dtype, const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                   const void* k, int64_t k_stride_token, int64_t k_stride_head, const void* v,
                                   int64_t v_stride_token, int64_t v_stride_head, void* q_out,
                                   int64_t q_out_stride_token, int64_t q_out_stride_head, const void* q_weight,
                                   const void* k_weight, float eps, const float* cos, const float* sin,
                                   int64_t rope_stride, int rope_rows, void* k_pool, void* v_pool,
                                   int64_t num_blocks, int n_heads, int n_kv_heads, int block_size, int head_dim,
                                   int64_t pool_stride_block, int64_t pool_stride_head, int64_t pool_stride_row,
                                   const int32_t* cu_seqlens, int num_seqs, int num_tokens, int max_q_len,
                                   const int32_t* positions, const int32_t* kv_page_tables, int num_pages_per_seq,
                                   int64_t table_stride, void* stream) {
    g_err.clear();
    const std::string f = "qk_norm_rope_cache_write";
    if (dtype != FEMTO_F32 && dtype != FEMTO_F16 && dtype != FEMTO_BF16)
        return fail(FEMTO_ERR_UNSUPPORTED, f + ": unsupported dtype " + std::to_string(dtype));
    if (head_dim != femto::kDimHead)
        return fail(FEMTO_ERR_UNSUPPORTED, f + ": head_dim must be " + std::to_string(femto::kDimHead));
    if (num_seqs < 0 || num_tokens < 0 || max_q_len < 0) return fail(FEMTO_ERR_INVALID, f + ": negative size");
    if (num_seqs == 0 || num_tokens == 0) return FEMTO_OK;
    if (!cu_seqlens && num_tokens != num_seqs)
        return fail(FEMTO_ERR_INVALID, f + ": without cu_seqlens every sequence has one token (num_tokens == num_seqs)");
    if (num_seqs > 65535) return fail(FEMTO_ERR_INVALID, f + ": at most 65535 sequences per call");
    if (block_size != femto::kPage)
        return fail(FEMTO_ERR_INVALID, f + ": block_size must be " + std::to_string(femto::kPage));
    if (n_heads <= 0 || n_kv_heads <= 0) return fail(FEMTO_ERR_INVALID, f + ": head counts must be positive");
    if (num_blocks < 1) return fail(FEMTO_ERR_INVALID, f + ": the pool needs at least one block");
    if (!(eps >= 0.0f)) return fail(FEMTO_ERR_INVALID, f + ": eps must be >= 0");
    if (!q || !k || !v || !q_out || !q_weight || !k_weight || !cos || !sin || !k_pool || !v_pool || !positions ||
        !kv_page_tables)
        return fail(FEMTO_ERR_INVALID, f + ": null pointer argument");
    if (rope_rows < 1 || rope_stride < femto::kDimHead) return fail(FEMTO_ERR_INVALID, f + ": rope tables too small");
    if (num_pages_per_seq < 0 || table_stride < num_pages_per_seq)
        return fail(FEMTO_ERR_INVALID, f + ": table stride smaller than its width");
    const int eb = elem_bytes(dtype);
    const void* ptrs[] = {q, k, v, q_out, q_weight, k_weight, k_pool, v_pool, cos, sin};
    for (const void* p : ptrs)
        if (!aligned(p, 16)) return fail(FEMTO_ERR_INVALID, f + ": tensors must be 16-byte aligned");
    const int64_t step = 16 / eb;
    if (q_stride_token % step || q_stride_head % step || k_stride_token % step || k_stride_head % step ||
        v_stride_token % step || v_stride_head % step || q_out_stride_token % step || q_out_stride_head % step ||
        pool_stride_block % step || pool_stride_head % step || pool_stride_row % step || rope_stride % 4)
        return fail(FEMTO_ERR_INVALID, f + ": strides must be multiples of 16 bytes");

    femto::PrologueArgs a{};
    femto::CacheWriteArgs& c = a.cw;
    c.k = k;
    c.v = v;
    c.k_stride_token = k_stride_token;
    c.k_stride_head = k_stride_head;
    c.v_stride_token = v_stride_token;
    c.v_stride_head = v_stride_head;
    c.k_pool = k_pool;
    c.v_pool = v_pool;
    c.num_blocks = num_blocks;
    c.pool_stride_block = pool_stride_block;
    c.pool_stride_head = pool_stride_head;
    c.pool_stride_row = pool_stride_row;
    c.cu_seqlens = cu_seqlens;
    c.positions = positions;
    c.tables = kv_page_tables;
    c.table_stride = table_stride;
    c.num_pages_per_seq = num_pages_per_seq;
    c.num_seqs = num_seqs;
    c.n_kv_heads = n_kv_heads;
    c.row_chunks = head_dim * eb / 16;
    c.elem_bytes = eb;
    a.q = q;
    a.q_stride_token = q_stride_token;
    a.q_stride_head = q_stride_head;
    a.q_out = q_out;
    a.q_out_stride_token = q_out_stride_token;
    a.q_out_stride_head = q_out_stride_head;
    a.q_weight = q_weight;
    a.k_weight = k_weight;
    a.eps = eps;
    a.cos = cos;
    a.sin = sin;
    a.rope_stride = rope_stride;
    a.rope_rows = rope_rows;
    a.positions_rope = positions;
    a.n_heads = n_heads;
    return hip_status(femto::launch_qk_norm_rope(dtype, a, cu_seqlens ? max_q_len : 1, static_cast<hipStream_t>(stream)),
                      "qk_norm_rope_cache_write launch");
}

int femto_build_varlen_metadata(int num_seqs, const int32_t* num_computed, const int32_t* num_tokens,
                                const int32_t* block_offsets, const int32_t* block_ids, int table_width,
                                int q_tile_size, int max_q_len, int32_t* positions, int32_t* cu_seqlens,
                                int32_t* cu_q_tiles, int32_t* q_tile_to_seq_idx, int32_t* kv_lens,
                                int32_t* block_tables, void* stream) {
    g_err.clear();
    const std::string f = "build_varlen_metadata";
    if (num_seqs < 0 || table_width < 0 || max_q_len < 0) return fail(FEMTO_ERR_INVALID, f + ": negative size");
    if (num_seqs == 0) return FEMTO_OK;
    if (num_seqs > 65535) return fail(FEMTO_ERR_INVALID, f + ": at most 65535 sequences per call");
    if (q_tile_size <= 0) return fail(FEMTO_ERR_INVALID, f + ": q_tile_size must be positive");
    if (!num_computed || !num_tokens || !block_offsets || !cu_seqlens || !cu_q_tiles || !kv_lens ||
        (table_width > 0 && (!block_ids || !block_tables)) || (max_q_len > 0 && (!positions || !q_tile_to_seq_idx)))
        return fail(FEMTO_ERR_INVALID, f + ": null pointer argument");
    femto::MetadataArgs a{};
    a.num_computed = num_computed;
    a.num_tokens = num_tokens;
    a.block_offsets = block_offsets;
    a.block_ids = block_ids;
    a.num_seqs = num_seqs;
    a.table_width = table_width;
    a.q_tile_size = q_tile_size;
    a.positions = positions;
    a.cu_seqlens = cu_seqlens;
    a.cu_q_tiles = cu_q_tiles;
    a.q_tile_to_seq_idx = q_tile_to_seq_idx;
    a.kv_lens = kv_lens;
    a.block_tables = block_tables;
    return hip_status(femto::launch_varlen_metadata(a, max_q_len, static_cast<hipStream_t>(stream)),
                      "build_varlen_metadata launch");
}

int femto_flash_attention(int dtype, const void* q, int64_t q_stride_batch, int64_t q_stride_head,
                          int64_t q_stride_token, const void* k, int64_t k_stride_batch, int64_t k_stride_head,
                          int64_t k_stride_token, const void* v, int64_t v_stride_batch, int64_t v_stride_head,
                          int64_t v_stride_token, void* out, int64_t out_stride_batch, int64_t out_stride_head,
                          int64_t out_stride_token, int batch, int n_heads, int n_kv_heads, int q_len, int kv_len,
                          int head_dim, void* stream) {
    g_err.clear();
    if (dtype != FEMTO_F16 && dtype != FEMTO_BF16)
        return fail(FEMTO_ERR_UNSUPPORTED, std::string("flash_attention: not implemented for '") + dtype_name(dtype) +
                                               "' (bf16 / f16 MFMA only)");
    if (head_dim != femto::kDimHead)
        return fail(FEMTO_ERR_UNSUPPORTED, "flash_attention: head_dim must be " + std::to_string(femto::kDimHead));
    if (batch < 0 || q_len < 0 || kv_len < 0) return fail(FEMTO_ERR_INVALID, "flash_attention: negative size");
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0)
        return fail(FEMTO_ERR_INVALID, "flash_attention: n_heads must be a positive multiple of n_kv_heads");
    if (batch == 0 || q_len == 0) return FEMTO_OK;
    if (!q || !k || !v || !out) return fail(FEMTO_ERR_INVALID, "flash_attention: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 8))
        return fail(FEMTO_ERR_INVALID, "flash_attention: q, k, v must be 16-byte aligned, out 8-byte aligned");
    const int64_t st[] = {q_stride_batch, q_stride_head, q_stride_token, k_stride_batch, k_stride_head,
                          k_stride_token, v_stride_batch, v_stride_head, v_stride_token};
    for (int64_t s : st)
        if (s % 8) return fail(FEMTO_ERR_INVALID, "flash_attention: q/k/v strides must be multiples of 16 bytes");
    if (out_stride_batch % 4 || out_stride_head % 4 || out_stride_token % 4)
        return fail(FEMTO_ERR_INVALID, "flash_attention: out strides must be multiples of 8 bytes");
    if (k_stride_token < 0 || k_stride_token > (1 << 24) || v_stride_token < 0 || v_stride_token > (1 << 24))
        return fail(FEMTO_ERR_INVALID, "flash_attention: k/v token stride out of range");

    femto::PrefillArgs a{};
    a.q = q;
    a.q_stride_batch = q_stride_batch;
    a.q_stride_head = q_stride_head;
    a.q_stride_token = q_stride_token;
    a.out = out;
    a.out_stride_batch = out_stride_batch;
    a.out_stride_head = out_stride_head;
    a.out_stride_token = out_stride_token;
    a.k = k;
    a.v = v;
    a.k_stride0 = k_stride_batch;
    a.k_stride1 = k_stride_head;
    a.k_stride2 = k_stride_token;
    a.v_stride0 = v_stride_batch;
    a.v_stride1 = v_stride_head;
    a.v_stride2 = v_stride_token;
    a.num_seqs = batch;
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.n_rep = n_heads / n_kv_heads;
    a.head_dim = head_dim;
    a.scale_log2 = scale_log2(head_dim);
    return hip_status(femto::launch_dense_attention(dtype, a, static_cast<hipStream_t>(stream)),
                      "flash_attention launch");
}

}  // extern "C"
