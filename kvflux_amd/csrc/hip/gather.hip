// Paged KV gather: BlockTable-driven read of whole pages into contiguous
// [token][head][dim] order. Same result as the reference's
// paged_kv_read_kernel (src/v2/paged_kv_read.cu:67-87): for sequence token
// t, head h, element d,
//   out[((off + t) * H + h) * D + d] = cache[((table[t / bs] * H + h) * bs + t % bs) * D + d]
// for K and V, generalised to many sequences per launch.
//
// gfx950 mapping. A page of one cache ([H][bs][D], H*bs*D elements) lands as
// one contiguous run of the output ([bs][H][D]: the same rows, (head, token)
// transposed at row granularity). A workgroup of 512 threads moves one part
// (1024 16-byte vectors, two per thread) of one (page, cache): thread
// vectors are numbered in OUTPUT order, so every
// wavefront store is 1 KiB contiguous and the part's dead vectors (tokens past
// a tail page's end) sit at its end; a part that starts past the tail exits
// before loading anything. Each thread issues its loads unconditionally (dead
// lanes reread vector 0 of the page) before its stores, which then go out
// back to back (loads under the store test serialise the stores: vmcnt counts
// both on gfx9).
//
// Memory policy and shape, measured on MI355X (64 sequences, L ~ U[512,
// 8192], 8 kv heads x 128 BF16, odd pages; launches back to back, kernel
// durations from rocprofv3):
//   * non-temporal loads and stores: each byte is read once and written once
//     (plain stores: 411-424 against 395 us for the live launch; 498 against
//     410 us for the table launch at one vector per thread);
//   * two 16-byte vectors per thread (one: 427-439 us, a whole page per
//     workgroup: 417 us);
//   * the (head, token) transposition costs 1.5% against a plain copy of
//     contiguous pages; the page-table lookup before the loads and the
//     random page placement cost about 3% each: an independent copy of the
//     same source pages into a contiguous buffer (no transposition,
//     kvflux_copy_page_list) runs at the same rate as this kernel.
//
// Two launches:
//   * kvflux_gather_paged_kv_live: one workgroup per (live page, part,
//     cache). The caller passes the exclusive scan of the per-sequence page
//     counts; each wavefront finds its sequence with a 64-ary search over it
//     (one ballot per level: one level up to 64 sequences, two up to 4096).
//   * kvflux_gather_paged_kv: the table-only form (no scan). A 2D grid of
//     (logical page x part, sequence, cache); workgroups past a sequence's end
//     exit after one metadata load (2.7% slower than the live launch on the
//     batch above, more when the lengths spread wider).
#include "common.h"

namespace kvflux_hip {
namespace {

constexpr int kThreads = 512;
constexpr int kLiveVpt = 2;   // vectors per thread, live-page launch
constexpr int kTableVpt = 2;  // vectors per thread, table launch

// Shape of one page and of one output token, in vectors.
struct PageShape {
    FastDiv token_vectors;  // H * vpr: vectors of one output token
    FastDiv row_vectors;    // vpr: vectors of one (head, token) row
    std::uint32_t block_size;
    std::uint32_t page_vectors;  // H * bs * vpr
};

// Part `part` of a page whose first `valid` tokens are live: src is the
// page's first vector in the cache, dst the page's first output vector.
template <typename Vec, int kVpt>
__device__ inline void gather_part(const Vec* __restrict__ src, Vec* __restrict__ dst, std::uint32_t valid,
                                   std::uint32_t part, const PageShape& shape) {
    const std::uint32_t live_vectors = valid * shape.token_vectors.divisor;
    const std::uint32_t first = part * (kThreads * kVpt);
    if (first >= live_vectors) return;  // uniform: the part lies past the tail
    const std::uint32_t vpr = shape.row_vectors.divisor;
    Vec r[kVpt];
    bool live[kVpt];
#pragma unroll
    for (int u = 0; u < kVpt; ++u) {
        const std::uint32_t j = first + u * kThreads + threadIdx.x;  // output order
        live[u] = j < live_vectors;
        const std::uint32_t token = shape.token_vectors.div(j);
        const std::uint32_t rest = j - token * shape.token_vectors.divisor;
        const std::uint32_t head = shape.row_vectors.div(rest);
        const std::uint32_t col = rest - head * vpr;
        const std::uint32_t s = (head * shape.block_size + token) * vpr + col;
        r[u] = stream_load(src + (live[u] ? s : 0u));
    }
#pragma unroll
    for (int u = 0; u < kVpt; ++u) keep_in_registers(r[u]);
#pragma unroll
    for (int u = 0; u < kVpt; ++u) {
        if (live[u]) stream_store(dst + first + u * kThreads + threadIdx.x, r[u]);
    }
}

// Last index i in [0, n) with starts[i] <= w, for a non-decreasing `starts`
// with starts[0] <= w (the sequence holding flat page w; empty sequences,
// whose start equals the next one's, are stepped over). Every lane of the
// wavefront takes part and gets the same answer: each level probes 64 evenly
// spaced entries and keeps the span between the last probe <= w and the next.
__device__ inline std::uint32_t find_sequence(const std::uint64_t* __restrict__ starts, std::uint32_t n,
                                              std::uint64_t w) {
    const std::uint32_t lane = threadIdx.x & 63u;
    std::uint32_t lo = 0;
    while (n > 1) {  // uniform
        const std::uint32_t step = (n + 63u) / 64u;
        const std::uint32_t k = lane * step;
        const bool below = k < n && starts[lo + k] <= w;
        std::uint32_t c = static_cast<std::uint32_t>(__popcll(__ballot(below)));
        if (c == 0) c = 1;  // starts[lo] > w only for a malformed scan: stay at lo
        lo += (c - 1u) * step;
        const std::uint32_t left = n - (c - 1u) * step;
        n = left < step ? left : step;
    }
    return lo;
}

template <typename Vec>
__global__ __launch_bounds__(kThreads) void paged_kv_gather_live_kernel(
    const Vec* __restrict__ key_cache, const Vec* __restrict__ value_cache, std::uint64_t num_blocks,
    const std::uint64_t* __restrict__ block_table, std::uint64_t table_width,
    const std::uint64_t* __restrict__ seq_lens, const std::uint64_t* __restrict__ out_offsets,
    const std::uint64_t* __restrict__ page_starts, std::uint32_t num_seqs, Vec* __restrict__ key_out,
    Vec* __restrict__ value_out, FastDiv parts, PageShape shape) {
    const std::uint32_t w = parts.div(blockIdx.x);
    const std::uint32_t part = blockIdx.x - w * parts.divisor;
    const std::uint32_t seq = __builtin_amdgcn_readfirstlane(find_sequence(page_starts, num_seqs, w));
    const std::uint64_t first_page = page_starts[seq];
    if (w < first_page) return;  // malformed scan
    const std::uint64_t logical = w - first_page;
    if (logical >= table_width) return;
    const std::uint64_t page = block_table[static_cast<std::uint64_t>(seq) * table_width + logical];
    const std::uint64_t length = seq_lens[seq];
    const std::uint64_t out_first = out_offsets[seq];
    const std::uint64_t first_token = logical * shape.block_size;
    if (first_token >= length || page >= num_blocks) return;  // padding or corrupt id: never dereferenced
    const std::uint64_t remaining = length - first_token;
    const std::uint32_t valid = remaining < shape.block_size ? static_cast<std::uint32_t>(remaining) : shape.block_size;
    const Vec* src = (blockIdx.z == 0 ? key_cache : value_cache) + page * shape.page_vectors;
    Vec* dst = (blockIdx.z == 0 ? key_out : value_out) + (out_first + first_token) * shape.token_vectors.divisor;
    gather_part<Vec, kLiveVpt>(src, dst, valid, part, shape);
}

template <typename Vec>
__global__ __launch_bounds__(kThreads) void paged_kv_gather_kernel(
    const Vec* __restrict__ key_cache, const Vec* __restrict__ value_cache, std::uint64_t num_blocks,
    const std::uint64_t* __restrict__ block_table, std::uint64_t table_width,
    const std::uint64_t* __restrict__ seq_lens, const std::uint64_t* __restrict__ out_offsets,
    std::uint32_t seq_base, Vec* __restrict__ key_out, Vec* __restrict__ value_out, FastDiv parts,
    PageShape shape) {
    const std::uint32_t seq = seq_base + blockIdx.y;
    const std::uint32_t logical = parts.div(blockIdx.x);  // < table_width (grid.x <= width * parts)
    const std::uint32_t part = blockIdx.x - logical * parts.divisor;
    // The three metadata loads are independent: issued together.
    const std::uint64_t page = block_table[static_cast<std::uint64_t>(seq) * table_width + logical];
    const std::uint64_t length = seq_lens[seq];
    const std::uint64_t out_first = out_offsets[seq];
    const std::uint64_t first_token = static_cast<std::uint64_t>(logical) * shape.block_size;
    if (first_token >= length || page >= num_blocks) return;
    const std::uint64_t remaining = length - first_token;
    const std::uint32_t valid = remaining < shape.block_size ? static_cast<std::uint32_t>(remaining) : shape.block_size;
    const Vec* src = (blockIdx.z == 0 ? key_cache : value_cache) + page * shape.page_vectors;
    Vec* dst = (blockIdx.z == 0 ? key_out : value_out) + (out_first + first_token) * shape.token_vectors.divisor;
    gather_part<Vec, kTableVpt>(src, dst, valid, part, shape);
}

// Validation shared by both entries; fills `shape` and the vector width.
int check_shape(const void* kc, const void* vc, std::uint64_t num_blocks, std::uint64_t heads,
                std::uint64_t block_size, std::uint64_t head_size, int dtype, const void* ko, const void* vo,
                unsigned* width, std::uint64_t* vpr_out, std::uint64_t* page_vectors_out) {
    const std::size_t esize = dtype_bytes(dtype);
    if (esize == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!kc || !vc || !ko || !vo) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: null pointer");
    if (num_blocks == 0 || heads == 0 || block_size == 0 || head_size == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: zero dimension");
    }
    if (heads > 0xffffffffULL || block_size > 0xffffffffULL || head_size > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged KV gather: page too large");
    }
    const std::uint64_t row_bytes = head_size * esize;
    const void* ptrs[4] = {kc, vc, ko, vo};
    *width = copy_width(row_bytes, ptrs, 4);
    if (*width < 2) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: misaligned buffers");
    const std::uint64_t vpr = row_bytes / *width;
    // Vector indices of a page stay below 2^32 with a part's worth to spare.
    const std::uint64_t limit = 0xffffffffULL - 2ULL * kThreads * kLiveVpt;
    if (vpr > limit || heads * block_size > limit / vpr) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged KV gather: page too large");
    }
    *vpr_out = vpr;
    *page_vectors_out = heads * block_size * vpr;
    return KVFLUX_OK;
}

PageShape make_shape(std::uint64_t heads, std::uint64_t block_size, std::uint64_t vpr) {
    PageShape s;
    s.token_vectors = FastDiv(static_cast<std::uint32_t>(heads * vpr));
    s.row_vectors = FastDiv(static_cast<std::uint32_t>(vpr));
    s.block_size = static_cast<std::uint32_t>(block_size);
    s.page_vectors = static_cast<std::uint32_t>(heads * block_size * vpr);
    return s;
}

template <typename Vec>
int launch_table(const void* kc, const void* vc, std::uint64_t num_blocks, const PageShape& shape,
                 const std::uint64_t* table, std::uint64_t width, const std::uint64_t* lens,
                 const std::uint64_t* offsets, std::uint64_t num_seqs, std::uint64_t max_len, void* ko, void* vo,
                 hipStream_t s) {
    std::uint64_t pages = (max_len + shape.block_size - 1) / shape.block_size;
    if (pages > width) pages = width;
    if (pages == 0) return KVFLUX_OK;
    const std::uint64_t parts = (shape.page_vectors + kThreads * kTableVpt - 1) / (kThreads * kTableVpt);
    if (pages * parts > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "gather: too many pages");
    for (std::uint64_t base = 0; base < num_seqs; base += 65535) {
        const std::uint64_t n = num_seqs - base < 65535 ? num_seqs - base : 65535;
        const dim3 grid(static_cast<unsigned>(pages * parts), static_cast<unsigned>(n), 2);
        hipLaunchKernelGGL(paged_kv_gather_kernel<Vec>, grid, dim3(kThreads), 0, s, static_cast<const Vec*>(kc),
                           static_cast<const Vec*>(vc), num_blocks, table, width, lens, offsets,
                           static_cast<std::uint32_t>(base), static_cast<Vec*>(ko), static_cast<Vec*>(vo),
                           FastDiv(static_cast<std::uint32_t>(parts)), shape);
        const int status = launch_status("paged_kv_gather_kernel");
        if (status != KVFLUX_OK) return status;
    }
    return KVFLUX_OK;
}

template <typename Vec>
int launch_live(const void* kc, const void* vc, std::uint64_t num_blocks, const PageShape& shape,
                const std::uint64_t* table, std::uint64_t width, const std::uint64_t* lens,
                const std::uint64_t* offsets, const std::uint64_t* starts, std::uint64_t num_seqs,
                std::uint64_t total_pages, void* ko, void* vo, hipStream_t s) {
    const std::uint64_t parts = (shape.page_vectors + kThreads * kLiveVpt - 1) / (kThreads * kLiveVpt);
    if (total_pages * parts > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "gather: too many pages");
    const dim3 grid(static_cast<unsigned>(total_pages * parts), 1, 2);
    hipLaunchKernelGGL(paged_kv_gather_live_kernel<Vec>, grid, dim3(kThreads), 0, s, static_cast<const Vec*>(kc),
                       static_cast<const Vec*>(vc), num_blocks, table, width, lens, offsets, starts,
                       static_cast<std::uint32_t>(num_seqs), static_cast<Vec*>(ko), static_cast<Vec*>(vo),
                       FastDiv(static_cast<std::uint32_t>(parts)), shape);
    return launch_status("paged_kv_gather_live_kernel");
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_gather_paged_kv(const void* key_cache, const void* value_cache,
                                      uint64_t num_blocks, uint64_t num_kv_heads,
                                      uint64_t block_size, uint64_t head_size, int dtype,
                                      const uint64_t* block_table, uint64_t max_blocks_per_seq,
                                      const uint64_t* seq_lens, const uint64_t* out_offsets,
                                      uint64_t num_seqs, uint64_t max_seq_len, void* key_out,
                                      void* value_out, void* stream) {
    if (num_seqs == 0 || max_seq_len == 0) return KVFLUX_OK;
    if (!block_table || !seq_lens || !out_offsets) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: null pointer");
    }
    unsigned width = 0;
    std::uint64_t vpr = 0, page_vectors = 0;
    int status = check_shape(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                             key_out, value_out, &width, &vpr, &page_vectors);
    if (status != KVFLUX_OK) return status;
    if (max_blocks_per_seq > 0xffffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "gather: table too wide");
    const PageShape shape = make_shape(num_kv_heads, block_size, vpr);
    const hipStream_t s = as_stream(stream);
    switch (width) {
    case 16: return launch_table<V16>(key_cache, value_cache, num_blocks, shape, block_table, max_blocks_per_seq,
                                      seq_lens, out_offsets, num_seqs, max_seq_len, key_out, value_out, s);
    case 8: return launch_table<V8>(key_cache, value_cache, num_blocks, shape, block_table, max_blocks_per_seq,
                                    seq_lens, out_offsets, num_seqs, max_seq_len, key_out, value_out, s);
    case 4: return launch_table<std::uint32_t>(key_cache, value_cache, num_blocks, shape, block_table,
                                               max_blocks_per_seq, seq_lens, out_offsets, num_seqs, max_seq_len,
                                               key_out, value_out, s);
    default: return launch_table<std::uint16_t>(key_cache, value_cache, num_blocks, shape, block_table,
                                                max_blocks_per_seq, seq_lens, out_offsets, num_seqs, max_seq_len,
                                                key_out, value_out, s);
    }
}

extern "C" int kvflux_gather_paged_kv_live(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                           uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size,
                                           int dtype, const uint64_t* block_table, uint64_t max_blocks_per_seq,
                                           const uint64_t* seq_lens, const uint64_t* out_offsets,
                                           const uint64_t* page_starts, uint64_t num_seqs, uint64_t total_pages,
                                           void* key_out, void* value_out, void* stream) {
    if (num_seqs == 0 || total_pages == 0) return KVFLUX_OK;
    if (!block_table || !seq_lens || !out_offsets || !page_starts) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: null pointer");
    }
    if (num_seqs > 0xffffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "gather: too many sequences");
    unsigned width = 0;
    std::uint64_t vpr = 0, page_vectors = 0;
    int status = check_shape(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                             key_out, value_out, &width, &vpr, &page_vectors);
    if (status != KVFLUX_OK) return status;
    const PageShape shape = make_shape(num_kv_heads, block_size, vpr);
    const hipStream_t s = as_stream(stream);
    switch (width) {
    case 16: return launch_live<V16>(key_cache, value_cache, num_blocks, shape, block_table, max_blocks_per_seq,
                                     seq_lens, out_offsets, page_starts, num_seqs, total_pages, key_out, value_out, s);
    case 8: return launch_live<V8>(key_cache, value_cache, num_blocks, shape, block_table, max_blocks_per_seq,
                                   seq_lens, out_offsets, page_starts, num_seqs, total_pages, key_out, value_out, s);
    case 4: return launch_live<std::uint32_t>(key_cache, value_cache, num_blocks, shape, block_table,
                                              max_blocks_per_seq, seq_lens, out_offsets, page_starts, num_seqs,
                                              total_pages, key_out, value_out, s);
    default: return launch_live<std::uint16_t>(key_cache, value_cache, num_blocks, shape, block_table,
                                               max_blocks_per_seq, seq_lens, out_offsets, page_starts, num_seqs,
                                               total_pages, key_out, value_out, s);
    }
}
