// Paged KV gather: BlockTable-driven read of whole pages into contiguous
// [token][head][dim] order. Same result as the reference's
// paged_kv_read_kernel (src/v2/paged_kv_read.cu:67-87): for sequence token
// t, head h, element d,
//   out[((off + t) * H + h) * D + d] = cache[((table[t / bs] * H + h) * bs + t % bs) * D + d]
// for K and V, generalised to many sequences per launch.
//
// gfx950 mapping: one 512-thread workgroup per (logical page, sequence,
// cache): blockIdx.z selects K (0) or V (1). A page of one cache is H*bs*D
// elements stored contiguously, so the workgroup streams it with consecutive
// lanes on consecutive 16-byte vectors (fully coalesced reads); each
// (head, token) row lands as one contiguous row of the output. Only the
// valid tokens of the tail page are touched. Every thread issues all of its
// loads, unconditionally (past the tail they reread vector 0 of the page),
// before its stores, which then go out back to back (with conditional loads
// each store waited for the previous one: 413 against 387 us for the
// 64-sequence BF16 batch on MI355X). Loads and stores carry the
// non-temporal hint: each byte is read once and written once (448 -> 415 us).
#include "common.h"

namespace kvflux_hip {
namespace {

constexpr int kThreads = 512;

template <typename Vec, int kMaxPerThread>
__global__ __launch_bounds__(kThreads) void paged_kv_gather_kernel(
    const Vec* __restrict__ key_cache, const Vec* __restrict__ value_cache,
    std::uint64_t num_blocks, const std::uint64_t* __restrict__ block_table,
    std::uint64_t table_width, const std::uint64_t* __restrict__ seq_lens,
    const std::uint64_t* __restrict__ out_offsets, Vec* __restrict__ key_out,
    Vec* __restrict__ value_out, std::uint32_t seq_base, FastDiv vectors_per_row,
    FastDiv block_size, std::uint32_t heads, std::uint32_t page_vectors) {
    const std::uint32_t seq = seq_base + blockIdx.y;
    const std::uint64_t logical = blockIdx.x;  // < table_width (grid.x <= width)
    // The three metadata loads are independent: issue them together.
    const std::uint64_t page = block_table[seq * table_width + logical];
    const std::uint64_t length = seq_lens[seq];
    const std::uint64_t out_first = out_offsets[seq];
    const std::uint64_t first_token = logical * block_size.divisor;
    if (first_token >= length) return;
    if (page >= num_blocks) return;  // padding or corrupt id: never dereference
    const std::uint64_t remaining = length - first_token;
    const std::uint32_t valid =
        remaining < block_size.divisor ? static_cast<std::uint32_t>(remaining) : block_size.divisor;

    const std::uint64_t src_base = page * page_vectors;
    const std::uint64_t out_token = out_first + first_token;
    const std::uint32_t vpr = vectors_per_row.divisor;

    const Vec* __restrict__ src = blockIdx.z == 0 ? key_cache : value_cache;
    Vec* __restrict__ out = blockIdx.z == 0 ? key_out : value_out;
    Vec k[kMaxPerThread];
    std::uint64_t dst[kMaxPerThread];
    bool live[kMaxPerThread];
#pragma unroll
    for (int u = 0; u < kMaxPerThread; ++u) {
        const std::uint32_t i = threadIdx.x + u * kThreads;  // vector within the page
        const std::uint32_t row = vectors_per_row.div(i);    // head * bs + token
        const std::uint32_t col = i - row * vpr;
        const std::uint32_t head = block_size.div(row);
        const std::uint32_t token = row - head * block_size.divisor;
        live[u] = i < page_vectors && token < valid;
        dst[u] = ((out_token + token) * heads + head) * vpr + col;
        k[u] = stream_load(src + src_base + (live[u] ? i : 0u));
    }
#pragma unroll
    for (int u = 0; u < kMaxPerThread; ++u) keep_in_registers(k[u]);
#pragma unroll
    for (int u = 0; u < kMaxPerThread; ++u) {
        if (live[u]) stream_store(out + dst[u], k[u]);
    }
}

// Pages larger than kThreads * 16 vectors: the same mapping in a loop
// (blockIdx.z selects the cache as above).
template <typename Vec>
__global__ __launch_bounds__(kThreads) void paged_kv_gather_kernel_loop(
    const Vec* __restrict__ key_cache, const Vec* __restrict__ value_cache,
    std::uint64_t num_blocks, const std::uint64_t* __restrict__ block_table,
    std::uint64_t table_width, const std::uint64_t* __restrict__ seq_lens,
    const std::uint64_t* __restrict__ out_offsets, Vec* __restrict__ key_out,
    Vec* __restrict__ value_out, std::uint32_t seq_base, std::uint64_t vpr,
    std::uint64_t block_size, std::uint64_t heads, std::uint64_t page_vectors) {
    const std::uint64_t seq = seq_base + blockIdx.y;
    const std::uint64_t logical = blockIdx.x;
    const std::uint64_t length = seq_lens[seq];
    const std::uint64_t first_token = logical * block_size;
    if (first_token >= length || logical >= table_width) return;
    const std::uint64_t page = block_table[seq * table_width + logical];
    if (page >= num_blocks) return;
    const std::uint64_t valid = length - first_token < block_size ? length - first_token : block_size;
    const std::uint64_t out_token = out_offsets[seq] + first_token;
    for (std::uint64_t i = threadIdx.x; i < page_vectors; i += kThreads) {
        const std::uint64_t row = i / vpr, col = i % vpr;
        const std::uint64_t head = row / block_size, token = row % block_size;
        if (token >= valid) continue;
        const std::uint64_t d = ((out_token + token) * heads + head) * vpr + col;
        if (blockIdx.z == 0) {
            stream_store(key_out + d, stream_load(key_cache + page * page_vectors + i));
        } else {
            stream_store(value_out + d, stream_load(value_cache + page * page_vectors + i));
        }
    }
}

template <typename Vec>
int launch(const void* kc, const void* vc, std::uint64_t num_blocks, std::uint64_t heads,
           std::uint64_t block_size, std::uint64_t row_bytes, const std::uint64_t* table,
           std::uint64_t width, const std::uint64_t* lens, const std::uint64_t* offsets,
           std::uint64_t num_seqs, std::uint64_t max_len, void* ko, void* vo, hipStream_t s) {
    const std::uint64_t vpr = row_bytes / sizeof(Vec);
    const std::uint64_t page_vectors = heads * block_size * vpr;
    std::uint64_t pages = (max_len + block_size - 1) / block_size;
    if (pages > width) pages = width;
    if (pages == 0) return KVFLUX_OK;
    if (pages > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "gather: too many pages");
    for (std::uint64_t base = 0; base < num_seqs; base += 65535) {
        const std::uint64_t n = num_seqs - base < 65535 ? num_seqs - base : 65535;
        const dim3 grid(static_cast<unsigned>(pages), static_cast<unsigned>(n), 2);
        if (page_vectors <= kThreads * 4) {
            hipLaunchKernelGGL((paged_kv_gather_kernel<Vec, 4>), grid, dim3(kThreads), 0, s,
                               static_cast<const Vec*>(kc), static_cast<const Vec*>(vc),
                               num_blocks, table, width, lens, offsets, static_cast<Vec*>(ko),
                               static_cast<Vec*>(vo), static_cast<std::uint32_t>(base),
                               FastDiv(static_cast<std::uint32_t>(vpr)),
                               FastDiv(static_cast<std::uint32_t>(block_size)),
                               static_cast<std::uint32_t>(heads),
                               static_cast<std::uint32_t>(page_vectors));
        } else if (page_vectors <= kThreads * 8) {
            hipLaunchKernelGGL((paged_kv_gather_kernel<Vec, 8>), grid, dim3(kThreads), 0, s,
                               static_cast<const Vec*>(kc), static_cast<const Vec*>(vc),
                               num_blocks, table, width, lens, offsets, static_cast<Vec*>(ko),
                               static_cast<Vec*>(vo), static_cast<std::uint32_t>(base),
                               FastDiv(static_cast<std::uint32_t>(vpr)),
                               FastDiv(static_cast<std::uint32_t>(block_size)),
                               static_cast<std::uint32_t>(heads),
                               static_cast<std::uint32_t>(page_vectors));
        } else if (page_vectors <= kThreads * 16) {
            hipLaunchKernelGGL((paged_kv_gather_kernel<Vec, 16>), grid, dim3(kThreads), 0, s,
                               static_cast<const Vec*>(kc), static_cast<const Vec*>(vc),
                               num_blocks, table, width, lens, offsets, static_cast<Vec*>(ko),
                               static_cast<Vec*>(vo), static_cast<std::uint32_t>(base),
                               FastDiv(static_cast<std::uint32_t>(vpr)),
                               FastDiv(static_cast<std::uint32_t>(block_size)),
                               static_cast<std::uint32_t>(heads),
                               static_cast<std::uint32_t>(page_vectors));
        } else {
            hipLaunchKernelGGL(paged_kv_gather_kernel_loop<Vec>, grid, dim3(kThreads), 0, s,
                               static_cast<const Vec*>(kc), static_cast<const Vec*>(vc),
                               num_blocks, table, width, lens, offsets, static_cast<Vec*>(ko),
                               static_cast<Vec*>(vo), static_cast<std::uint32_t>(base), vpr,
                               block_size, heads, page_vectors);
        }
        const int status = launch_status("paged_kv_gather_kernel");
        if (status != KVFLUX_OK) return status;
    }
    return KVFLUX_OK;
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
    const std::size_t esize = dtype_bytes(dtype);
    if (esize == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!key_cache || !value_cache || !block_table || !seq_lens || !out_offsets || !key_out ||
        !value_out) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: null pointer");
    }
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: zero dimension");
    }
    const std::uint64_t row_bytes = head_size * esize;
    const std::uint64_t page_rows = num_kv_heads * block_size;
    if (page_rows > 0xffffffffULL || row_bytes > 0xffffffffULL ||
        page_rows * (row_bytes / 2 + 1) > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged KV gather: page too large");
    }
    const void* ptrs[4] = {key_cache, value_cache, key_out, value_out};
    const unsigned width = copy_width(row_bytes, ptrs, 4);
    const hipStream_t s = as_stream(stream);
    switch (width) {
    case 16: return launch<V16>(key_cache, value_cache, num_blocks, num_kv_heads, block_size,
                                row_bytes, block_table, max_blocks_per_seq, seq_lens, out_offsets,
                                num_seqs, max_seq_len, key_out, value_out, s);
    case 8: return launch<V8>(key_cache, value_cache, num_blocks, num_kv_heads, block_size,
                              row_bytes, block_table, max_blocks_per_seq, seq_lens, out_offsets,
                              num_seqs, max_seq_len, key_out, value_out, s);
    case 4: return launch<std::uint32_t>(key_cache, value_cache, num_blocks, num_kv_heads,
                                         block_size, row_bytes, block_table, max_blocks_per_seq,
                                         seq_lens, out_offsets, num_seqs, max_seq_len, key_out,
                                         value_out, s);
    case 2: return launch<std::uint16_t>(key_cache, value_cache, num_blocks, num_kv_heads,
                                         block_size, row_bytes, block_table, max_blocks_per_seq,
                                         seq_lens, out_offsets, num_seqs, max_seq_len, key_out,
                                         value_out, s);
    default: return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV gather: misaligned buffers");
    }
}
