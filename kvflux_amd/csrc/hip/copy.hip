// Batched page copy: copy-on-write of shared pages for many sequences in one
// launch. The reference copies one page per call with two cudaMemcpyAsync
// (K page, V page) and a synchronisation (src/v2/paged_kv_storage.cpp:70-93);
// here every (source, destination) pair of a decode step is one kernel:
//   K[dst][*] = K[src][*],  V[dst][*] = V[src][*]
// where a page holds all kv heads contiguously (page_bytes = H * bs * D * e,
// layout K/V[num_blocks][H][bs][D]). Raw bit copy.
//
// gfx950 mapping: grid (pair, 16 KiB part of the page, K or V). A workgroup of
// 512 threads moves its part with 16-byte loads, all issued (unconditionally)
// before the stores, which then go out back to back, so one wavefront
// streams 1 KiB contiguous per instruction. The pair
// is read once per workgroup (uniform, scalar loads).
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
constexpr std::uint64_t kPartBytes = 16384;  // bytes of a page per workgroup

// Part blockIdx.y of an n-vector range: every load issued before the stores,
// both with the non-temporal hint (each byte moves once).
template <typename Vec>
__device__ inline void copy_part(const Vec* __restrict__ from, Vec* __restrict__ to, std::uint64_t n) {
    constexpr int kPer = static_cast<int>(kPartBytes / sizeof(Vec) / kCopyThreads);
    const std::uint64_t first = static_cast<std::uint64_t>(blockIdx.y) * (kPartBytes / sizeof(Vec)) + threadIdx.x;
    Vec r[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const std::uint64_t i = first + static_cast<std::uint64_t>(u) * kCopyThreads;
        r[u] = stream_load(from + (i < n ? i : 0));  // n >= 1: vector 0 is in range
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) keep_in_registers(r[u]);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const std::uint64_t i = first + static_cast<std::uint64_t>(u) * kCopyThreads;
        if (i < n) stream_store(to + i, r[u]);
    }
}

template <typename Vec>
__global__ __launch_bounds__(kCopyThreads) void copy_pages_kernel(char* __restrict__ key_cache,
                                                                  char* __restrict__ value_cache,
                                                                  std::uint64_t num_blocks,
                                                                  std::uint64_t page_bytes,
                                                                  const std::uint64_t* __restrict__ pairs) {
    const std::uint64_t src = pairs[2 * static_cast<std::uint64_t>(blockIdx.x)];
    const std::uint64_t dst = pairs[2 * static_cast<std::uint64_t>(blockIdx.x) + 1];
    if (src >= num_blocks || dst >= num_blocks || src == dst) return;  // uniform
    char* base = blockIdx.z == 0 ? key_cache : value_cache;
    copy_part(reinterpret_cast<const Vec*>(base + src * page_bytes), reinterpret_cast<Vec*>(base + dst * page_bytes),
              page_bytes / sizeof(Vec));
}

template <typename Vec>
int launch_copy(void* kc, void* vc, std::uint64_t num_blocks, std::uint64_t page_bytes,
                const std::uint64_t* pairs, std::uint64_t num_pairs, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(num_pairs),
                    static_cast<unsigned>((page_bytes + kPartBytes - 1) / kPartBytes), 2);
    hipLaunchKernelGGL(copy_pages_kernel<Vec>, grid, dim3(kCopyThreads), 0, s, static_cast<char*>(kc),
                       static_cast<char*>(vc), num_blocks, page_bytes, pairs);
    return launch_status("copy_pages_kernel");
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
    if (num_pairs > 0x7fffffffULL || (page_bytes + kPartBytes - 1) / kPartBytes > 65535) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "copy pages: more than 2^31 pairs or pages above 1 GiB");
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
