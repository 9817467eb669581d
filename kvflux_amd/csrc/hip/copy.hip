// Batched page copy: copy-on-write of shared pages for many sequences in one
// launch. The reference copies one page per call with two cudaMemcpyAsync
// (K page, V page) and a synchronisation (src/v2/paged_kv_storage.cpp:70-93);
// here every (source, destination) pair of a decode step is one kernel:
//   K[dst][*] = K[src][*],  V[dst][*] = V[src][*]
// where a page holds all kv heads contiguously (page_bytes = H * bs * D * e,
// layout K/V[num_blocks][H][bs][D]). Raw bit copy.
//
// gfx950 mapping: grid (pair x part, K or V), the part index fastest, so the
// workgroups of one page are dispatched together. A workgroup of 512 threads
// moves one part of 512 vectors (8 KiB with 16-byte vectors), one vector per
// thread, with non-temporal loads and stores (each byte moves once).
// Measured on MI355X, 4096 pairs of random 32 KiB pages of a 65536-page
// arena (0.537 GB moved), eight rotated pair sets covering the arena,
// launches back to back, kernel durations from rocprofv3: 106-108 us for
// every part size from 8 to 32 KiB and 256 to 1024 threads; plain stores
// 111 us; contiguous pairs 77 us. The random page placement, not the copy
// loop, sets the rate (with a sync between launches the Infinity Cache
// drains plain stores in the gaps and hides part of that: 91 us, not an HBM
// rate).
//
// The same part copy moves KV chunks between the GPU and pinned host memory
// (offload / onload): kvflux_copy_chunks takes (source, destination) address
// pairs, so a batch of chunks whose host slots are scattered is one launch
// instead of one cudaMemcpyAsync per chunk (reference
// src/v3/gpu_cpu_transfer.cpp:32-95).
#include "common.h"

namespace kvflux_hip {
namespace {

constexpr int kCopyThreads = 512;
constexpr std::uint64_t kPartBytes = 16384;  // bytes of a chunk per workgroup step (kvflux_copy_chunks)

template <typename Vec>
__global__ __launch_bounds__(kCopyThreads) void copy_pages_kernel(char* __restrict__ key_cache,
                                                                  char* __restrict__ value_cache,
                                                                  std::uint64_t num_blocks,
                                                                  std::uint64_t page_bytes, FastDiv parts,
                                                                  const std::uint64_t* __restrict__ pairs) {
    const std::uint32_t pair = parts.div(blockIdx.x);
    const std::uint32_t part = blockIdx.x - pair * parts.divisor;
    const std::uint64_t src = pairs[2 * static_cast<std::uint64_t>(pair)];
    const std::uint64_t dst = pairs[2 * static_cast<std::uint64_t>(pair) + 1];
    if (src >= num_blocks || dst >= num_blocks || src == dst) return;  // uniform
    char* base = blockIdx.y == 0 ? key_cache : value_cache;
    const std::uint64_t n = page_bytes / sizeof(Vec);
    const std::uint64_t i = static_cast<std::uint64_t>(part) * kCopyThreads + threadIdx.x;
    if (i < n) {
        const Vec v = stream_load(reinterpret_cast<const Vec*>(base + src * page_bytes) + i);
        stream_store(reinterpret_cast<Vec*>(base + dst * page_bytes) + i, v);
    }
}

template <typename Vec>
int launch_copy(void* kc, void* vc, std::uint64_t num_blocks, std::uint64_t page_bytes,
                const std::uint64_t* pairs, std::uint64_t num_pairs, hipStream_t s) {
    const std::uint64_t parts = (page_bytes / sizeof(Vec) + kCopyThreads - 1) / kCopyThreads;
    if (num_pairs * parts > 0x7fffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "copy pages: more than 2^31 page parts in one call");
    }
    const dim3 grid(static_cast<unsigned>(num_pairs * parts), 2);
    hipLaunchKernelGGL(copy_pages_kernel<Vec>, grid, dim3(kCopyThreads), 0, s, static_cast<char*>(kc),
                       static_cast<char*>(vc), num_blocks, page_bytes, FastDiv(static_cast<std::uint32_t>(parts)),
                       pairs);
    return launch_status("copy_pages_kernel");
}

// Page-list copy: page i of `dst` = page src_pages[i] of `src` (pages of
// page_bytes; ids >= num_src_blocks are skipped). A gather of whole pages
// into a contiguous buffer with no reordering inside a page: staging of a
// sequence's pages for a transfer, and the independent copy that reads the
// same fragmented pages as the KV gather. Same part mapping as
// copy_pages_kernel, one cache per call.
template <typename Vec>
__global__ __launch_bounds__(kCopyThreads) void copy_page_list_kernel(char* __restrict__ dst,
                                                                      const char* __restrict__ src,
                                                                      std::uint64_t num_src_blocks,
                                                                      std::uint64_t page_bytes, FastDiv parts,
                                                                      const std::uint64_t* __restrict__ src_pages) {
    const std::uint32_t page = parts.div(blockIdx.x);
    const std::uint32_t part = blockIdx.x - page * parts.divisor;
    const std::uint64_t from = src_pages[page];
    if (from >= num_src_blocks) return;  // uniform
    const std::uint64_t n = page_bytes / sizeof(Vec);
    const std::uint64_t i = static_cast<std::uint64_t>(part) * kCopyThreads + threadIdx.x;
    if (i < n) {
        const Vec v = stream_load(reinterpret_cast<const Vec*>(src + from * page_bytes) + i);
        stream_store(reinterpret_cast<Vec*>(dst + static_cast<std::uint64_t>(page) * page_bytes) + i, v);
    }
}

template <typename Vec>
int launch_page_list(void* dst, const void* src, std::uint64_t num_src_blocks, std::uint64_t page_bytes,
                     const std::uint64_t* src_pages, std::uint64_t num_pages, hipStream_t s) {
    const std::uint64_t parts = (page_bytes / sizeof(Vec) + kCopyThreads - 1) / kCopyThreads;
    if (num_pages * parts > 0x7fffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "copy page list: more than 2^31 page parts in one call");
    }
    hipLaunchKernelGGL(copy_page_list_kernel<Vec>, dim3(static_cast<unsigned>(num_pages * parts)), dim3(kCopyThreads),
                       0, s, static_cast<char*>(dst), static_cast<const char*>(src), num_src_blocks, page_bytes,
                       FastDiv(static_cast<std::uint32_t>(parts)), src_pages);
    return launch_status("copy_page_list_kernel");
}

// Batched chunk copy between arbitrary device-visible addresses (device
// memory, or pinned host memory mapped into the device address space). The
// host link, not HBM, bounds these copies, so a bounded grid walks the
// (pair, 16 KiB part) items: 64 workgroups keep about 1 MiB of 16-byte
// requests in flight, which fills the link (measured on MI355X: 55 GB/s
// device -> host, 57 GB/s host -> device, the same as with 1024), while
// disturbing an HBM-bound kernel on another stream less than a wide grid
// does.
constexpr unsigned kChunkGrid = 64;

template <typename Vec>
__global__ __launch_bounds__(kCopyThreads) void copy_chunks_kernel(const std::uint64_t* __restrict__ pairs,
                                                                   std::uint64_t num_pairs, std::uint64_t parts,
                                                                   std::uint64_t chunk_bytes) {
    constexpr int kPer = static_cast<int>(kPartBytes / sizeof(Vec) / kCopyThreads);
    const std::uint64_t n = chunk_bytes / sizeof(Vec);
    for (std::uint64_t item = blockIdx.x; item < num_pairs * parts; item += gridDim.x) {  // uniform
        const std::uint64_t pair = item / parts, part = item % parts;
        const auto* from = reinterpret_cast<const Vec*>(pairs[2 * pair]);
        auto* to = reinterpret_cast<Vec*>(pairs[2 * pair + 1]);
        const std::uint64_t first = part * (kPartBytes / sizeof(Vec)) + threadIdx.x;
        Vec r[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const std::uint64_t i = first + static_cast<std::uint64_t>(u) * kCopyThreads;
            r[u] = from[i < n ? i : 0];  // n >= 1: vector 0 is in range
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) keep_in_registers(r[u]);
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const std::uint64_t i = first + static_cast<std::uint64_t>(u) * kCopyThreads;
            if (i < n) to[i] = r[u];
        }
    }
}

template <typename Vec>
int launch_chunks(const std::uint64_t* pairs, std::uint64_t num_pairs, std::uint64_t chunk_bytes, hipStream_t s) {
    const std::uint64_t parts = (chunk_bytes + kPartBytes - 1) / kPartBytes;
    const std::uint64_t items = num_pairs * parts;
    const unsigned grid = static_cast<unsigned>(items < kChunkGrid ? items : kChunkGrid);
    hipLaunchKernelGGL(copy_chunks_kernel<Vec>, dim3(grid), dim3(kCopyThreads), 0, s, pairs, num_pairs, parts,
                       chunk_bytes);
    return launch_status("copy_chunks_kernel");
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_copy_chunks(const uint64_t* pairs, uint64_t num_pairs, uint64_t chunk_bytes, void* stream) {
    if (num_pairs == 0 || chunk_bytes == 0) return KVFLUX_OK;
    if (!pairs) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "copy chunks: null pointer");
    if (num_pairs > (~0ULL) / ((chunk_bytes + kPartBytes - 1) / kPartBytes)) {
        return fail(KVFLUX_ERR_OVERFLOW, "copy chunks: size overflow");
    }
    const hipStream_t s = as_stream(stream);
    switch (copy_width(chunk_bytes, nullptr, 0)) {
    case 16: return launch_chunks<V16>(pairs, num_pairs, chunk_bytes, s);
    case 8: return launch_chunks<V8>(pairs, num_pairs, chunk_bytes, s);
    case 4: return launch_chunks<std::uint32_t>(pairs, num_pairs, chunk_bytes, s);
    case 2: return launch_chunks<std::uint16_t>(pairs, num_pairs, chunk_bytes, s);
    default: return launch_chunks<std::uint8_t>(pairs, num_pairs, chunk_bytes, s);
    }
}

extern "C" int kvflux_copy_pages(void* key_cache, void* value_cache, uint64_t num_blocks,
                                 uint64_t page_bytes, const uint64_t* pairs, uint64_t num_pairs,
                                 void* stream) {
    if (num_pairs == 0) return KVFLUX_OK;
    if (!key_cache || !value_cache || !pairs) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "copy pages: null pointer");
    if (num_blocks == 0 || page_bytes == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "copy pages: zero dimension");
    if (num_blocks > (~0ULL) / page_bytes) return fail(KVFLUX_ERR_OVERFLOW, "copy pages: size overflow");
    if (num_pairs > 0x7fffffffULL || page_bytes / kCopyThreads > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "copy pages: more than 2^31 pairs or pages above 2 TiB");
    }
    const void* ptrs[2] = {key_cache, value_cache};
    const hipStream_t s = as_stream(stream);
    switch (copy_width(page_bytes, ptrs, 2)) {
    case 16: return launch_copy<V16>(key_cache, value_cache, num_blocks, page_bytes, pairs, num_pairs, s);
    case 8: return launch_copy<V8>(key_cache, value_cache, num_blocks, page_bytes, pairs, num_pairs, s);
    case 4: return launch_copy<std::uint32_t>(key_cache, value_cache, num_blocks, page_bytes, pairs, num_pairs, s);
    case 2: return launch_copy<std::uint16_t>(key_cache, value_cache, num_blocks, page_bytes, pairs, num_pairs, s);
    default: return launch_copy<std::uint8_t>(key_cache, value_cache, num_blocks, page_bytes, pairs, num_pairs, s);
    }
}

extern "C" int kvflux_copy_page_list(void* dst, const void* src, uint64_t num_src_blocks, uint64_t page_bytes,
                                     const uint64_t* src_pages, uint64_t num_pages, void* stream) {
    if (num_pages == 0) return KVFLUX_OK;
    if (!dst || !src || !src_pages) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "copy page list: null pointer");
    if (num_src_blocks == 0 || page_bytes == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "copy page list: zero dimension");
    }
    if (num_src_blocks > (~0ULL) / page_bytes || num_pages > (~0ULL) / page_bytes) {
        return fail(KVFLUX_ERR_OVERFLOW, "copy page list: size overflow");
    }
    if (num_pages > 0x7fffffffULL || page_bytes / kCopyThreads > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "copy page list: more than 2^31 pages or pages above 2 TiB");
    }
    const void* ptrs[2] = {dst, src};
    const hipStream_t s = as_stream(stream);
    switch (copy_width(page_bytes, ptrs, 2)) {
    case 16: return launch_page_list<V16>(dst, src, num_src_blocks, page_bytes, src_pages, num_pages, s);
    case 8: return launch_page_list<V8>(dst, src, num_src_blocks, page_bytes, src_pages, num_pages, s);
    case 4: return launch_page_list<std::uint32_t>(dst, src, num_src_blocks, page_bytes, src_pages, num_pages, s);
    case 2: return launch_page_list<std::uint16_t>(dst, src, num_src_blocks, page_bytes, src_pages, num_pages, s);
    default: return launch_page_list<std::uint8_t>(dst, src, num_src_blocks, page_bytes, src_pages, num_pages, s);
    }
}
