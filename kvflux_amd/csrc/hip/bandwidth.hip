// HBM bandwidth probe: plain streaming copy, write-only and read-only
// kernels over one contiguous range, with the launch shape as a parameter
// (threads per workgroup, 16-byte vectors per thread, grid, non-temporal or
// plain accesses). These are the ceilings the data-path kernels are judged
// against: a kernel that moves the same bytes with no page table, no
// transposition and no fragmentation.
//
// Shape: a workgroup step moves threads * vectors_per_thread consecutive
// 16-byte vectors; thread t takes vectors t, t + threads, ... of the step, so
// every wavefront access is 1 KiB contiguous. grid == 0 launches one
// workgroup per step (one-shot); otherwise `grid` workgroups walk the steps
// (grid-stride). A thread issues all its loads before its stores.
//
// A second probe reads a list of pages of two caches (K and V) and nothing
// else: the read ceiling of a kernel that must visit the same scattered pages
// in the same order (the batch decode's unique pages), one workgroup per
// (page part, cache), one-shot.
#include "common.h"

namespace kvflux_hip {
namespace {

template <bool kNt>
__device__ inline V16 probe_load(const V16* p) {
    if constexpr (kNt) return stream_load(p);
    else return *p;
}
template <bool kNt>
__device__ inline void probe_store(V16* p, const V16& v) {
    if constexpr (kNt) stream_store(p, v);
    else *p = v;
}

template <int kT, int kVpt, bool kNt>
__global__ __launch_bounds__(kT) void probe_copy_kernel(const V16* __restrict__ src, V16* __restrict__ dst,
                                                         std::uint64_t steps) {
    for (std::uint64_t c = blockIdx.x; c < steps; c += gridDim.x) {
        const std::uint64_t b = c * (kT * kVpt) + threadIdx.x;
        V16 r[kVpt];
#pragma unroll
        for (int u = 0; u < kVpt; ++u) r[u] = probe_load<kNt>(src + b + u * kT);
#pragma unroll
        for (int u = 0; u < kVpt; ++u) keep_in_registers(r[u]);
#pragma unroll
        for (int u = 0; u < kVpt; ++u) probe_store<kNt>(dst + b + u * kT, r[u]);
    }
}

template <int kT, int kVpt, bool kNt>
__global__ __launch_bounds__(kT) void probe_write_kernel(V16* __restrict__ dst, std::uint64_t steps) {
    const V16 v{{0x6b766678u, 0x75782031u, 0x6b766678u ^ threadIdx.x, 0x75782032u}};
    for (std::uint64_t c = blockIdx.x; c < steps; c += gridDim.x) {
        const std::uint64_t b = c * (kT * kVpt) + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kVpt; ++u) probe_store<kNt>(dst + b + u * kT, v);
    }
}

// Read-only: the loaded words are folded into one xor per thread, written to
// sink[threadIdx.x] only when it equals a fixed pattern (so the loads stay
// live and the sink, of kT vectors, is almost never touched).
template <int kT, int kVpt, bool kNt>
__global__ __launch_bounds__(kT) void probe_read_kernel(const V16* __restrict__ src, std::uint64_t steps,
                                                         V16* __restrict__ sink) {
    V16 acc{{0u, 0u, 0u, 0u}};
    for (std::uint64_t c = blockIdx.x; c < steps; c += gridDim.x) {
        const std::uint64_t b = c * (kT * kVpt) + threadIdx.x;
        V16 r[kVpt];
#pragma unroll
        for (int u = 0; u < kVpt; ++u) r[u] = probe_load<kNt>(src + b + u * kT);
#pragma unroll
        for (int u = 0; u < kVpt; ++u) {
            for (int k = 0; k < 4; ++k) acc.w[k] ^= r[u].w[k];
        }
    }
    if (acc.w[0] == 0x9e3779b9u && acc.w[1] == 0x7f4a7c15u && acc.w[2] == 0x85ebca6bu) sink[threadIdx.x] = acc;
}

// Read-only over pages: workgroup (item, cache) reads part item % parts of
// page pages[item / parts] (kT * kVpt vectors; ids >= num_blocks are
// skipped), folding the words into the sink test of probe_read_kernel.
template <int kT, int kVpt, bool kNt>
__global__ __launch_bounds__(kT) void probe_read_pages_kernel(const V16* __restrict__ key_cache,
                                                               const V16* __restrict__ value_cache,
                                                               std::uint64_t num_blocks, std::uint64_t page_vectors,
                                                               FastDiv parts, const std::uint64_t* __restrict__ pages,
                                                               V16* __restrict__ sink) {
    const std::uint32_t index = parts.div(blockIdx.x);
    const std::uint32_t part = blockIdx.x - index * parts.divisor;
    const std::uint64_t page = pages[index];
    if (page >= num_blocks) return;  // uniform
    const V16* src = (blockIdx.y == 0 ? key_cache : value_cache) + page * page_vectors +
                     static_cast<std::uint64_t>(part) * (kT * kVpt) + threadIdx.x;
    V16 r[kVpt];
#pragma unroll
    for (int u = 0; u < kVpt; ++u) r[u] = probe_load<kNt>(src + u * kT);
    V16 acc{{0u, 0u, 0u, 0u}};
#pragma unroll
    for (int u = 0; u < kVpt; ++u) {
        for (int k = 0; k < 4; ++k) acc.w[k] ^= r[u].w[k];
    }
    if (acc.w[0] == 0x9e3779b9u && acc.w[1] == 0x7f4a7c15u && acc.w[2] == 0x85ebca6bu) sink[threadIdx.x] = acc;
}

template <int kT, int kVpt>
int probe_pages_launch(const void* kc, const void* vc, std::uint64_t num_blocks, std::uint64_t page_vectors,
                       const std::uint64_t* pages, std::uint64_t num_pages, int nt, void* sink, hipStream_t s) {
    const std::uint64_t parts = page_vectors / (kT * kVpt);
    const dim3 grid(static_cast<unsigned>(num_pages * parts), 2);
    if (nt) {
        hipLaunchKernelGGL((probe_read_pages_kernel<kT, kVpt, true>), grid, dim3(kT), 0, s,
                           static_cast<const V16*>(kc), static_cast<const V16*>(vc), num_blocks, page_vectors,
                           FastDiv(static_cast<std::uint32_t>(parts)), pages, static_cast<V16*>(sink));
    } else {
        hipLaunchKernelGGL((probe_read_pages_kernel<kT, kVpt, false>), grid, dim3(kT), 0, s,
                           static_cast<const V16*>(kc), static_cast<const V16*>(vc), num_blocks, page_vectors,
                           FastDiv(static_cast<std::uint32_t>(parts)), pages, static_cast<V16*>(sink));
    }
    return launch_status("bandwidth page probe kernel");
}

template <int kT>
int probe_pages_vpt(const void* kc, const void* vc, std::uint64_t num_blocks, std::uint64_t page_vectors,
                    const std::uint64_t* pages, std::uint64_t num_pages, unsigned vpt, int nt, void* sink,
                    hipStream_t s) {
    switch (vpt) {
    case 1: return probe_pages_launch<kT, 1>(kc, vc, num_blocks, page_vectors, pages, num_pages, nt, sink, s);
    case 2: return probe_pages_launch<kT, 2>(kc, vc, num_blocks, page_vectors, pages, num_pages, nt, sink, s);
    case 4: return probe_pages_launch<kT, 4>(kc, vc, num_blocks, page_vectors, pages, num_pages, nt, sink, s);
    default: return probe_pages_launch<kT, 8>(kc, vc, num_blocks, page_vectors, pages, num_pages, nt, sink, s);
    }
}

template <int kT, int kVpt, bool kNt>
int probe_launch(int op, void* dst, const void* src, std::uint64_t steps, unsigned grid, hipStream_t s) {
    switch (op) {
    case 0:
        hipLaunchKernelGGL((probe_copy_kernel<kT, kVpt, kNt>), dim3(grid), dim3(kT), 0, s,
                           static_cast<const V16*>(src), static_cast<V16*>(dst), steps);
        break;
    case 1:
        hipLaunchKernelGGL((probe_write_kernel<kT, kVpt, kNt>), dim3(grid), dim3(kT), 0, s, static_cast<V16*>(dst),
                           steps);
        break;
    default:
        hipLaunchKernelGGL((probe_read_kernel<kT, kVpt, kNt>), dim3(grid), dim3(kT), 0, s,
                           static_cast<const V16*>(src), steps, static_cast<V16*>(dst));
        break;
    }
    return launch_status("bandwidth probe kernel");
}

template <int kT, int kVpt>
int probe_nt(int op, void* dst, const void* src, std::uint64_t steps, unsigned grid, int nt, hipStream_t s) {
    return nt ? probe_launch<kT, kVpt, true>(op, dst, src, steps, grid, s)
              : probe_launch<kT, kVpt, false>(op, dst, src, steps, grid, s);
}

template <int kT>
int probe_vpt(int op, void* dst, const void* src, std::uint64_t steps, unsigned grid, unsigned vpt, int nt,
              hipStream_t s) {
    switch (vpt) {
    case 1: return probe_nt<kT, 1>(op, dst, src, steps, grid, nt, s);
    case 2: return probe_nt<kT, 2>(op, dst, src, steps, grid, nt, s);
    case 4: return probe_nt<kT, 4>(op, dst, src, steps, grid, nt, s);
    default: return probe_nt<kT, 8>(op, dst, src, steps, grid, nt, s);
    }
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_bandwidth_probe(int op, void* dst, const void* src, uint64_t bytes, uint32_t threads,
                                      uint32_t vectors_per_thread, uint32_t grid, int nontemporal, void* stream) {
    if (op < 0 || op > 2) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: op is 0 (copy), 1 (write) or 2 (read)");
    if (threads != 256 && threads != 512 && threads != 1024) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: threads is 256, 512 or 1024");
    }
    if (vectors_per_thread != 1 && vectors_per_thread != 2 && vectors_per_thread != 4 && vectors_per_thread != 8) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: vectors_per_thread is 1, 2, 4 or 8");
    }
    const std::uint64_t step_bytes = 16ULL * threads * vectors_per_thread;
    if (bytes == 0 || bytes % step_bytes != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: bytes must be a positive multiple of %llu",
                    static_cast<unsigned long long>(step_bytes));
    }
    // dst: the copy or write target, or the read sink (threads * 16 bytes).
    if (!dst || (op != 1 && !src)) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: null pointer");
    if ((reinterpret_cast<std::uintptr_t>(dst) | reinterpret_cast<std::uintptr_t>(src)) % 16 != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth probe: buffers must be 16-byte aligned");
    }
    const std::uint64_t steps = bytes / step_bytes;
    const std::uint64_t blocks = grid == 0 ? steps : (grid < steps ? grid : steps);
    if (blocks > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "bandwidth probe: grid too large");
    const hipStream_t s = as_stream(stream);
    const auto g = static_cast<unsigned>(blocks);
    switch (threads) {
    case 256: return probe_vpt<256>(op, dst, src, steps, g, vectors_per_thread, nontemporal, s);
    case 512: return probe_vpt<512>(op, dst, src, steps, g, vectors_per_thread, nontemporal, s);
    default: return probe_vpt<1024>(op, dst, src, steps, g, vectors_per_thread, nontemporal, s);
    }
}

extern "C" int kvflux_bandwidth_probe_pages(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                            uint64_t page_bytes, const uint64_t* pages, uint64_t num_pages,
                                            uint32_t threads, uint32_t vectors_per_thread, int nontemporal,
                                            void* sink, void* stream) {
    if (threads != 256 && threads != 512 && threads != 1024) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth page probe: threads is 256, 512 or 1024");
    }
    if (vectors_per_thread != 1 && vectors_per_thread != 2 && vectors_per_thread != 4 && vectors_per_thread != 8) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth page probe: vectors_per_thread is 1, 2, 4 or 8");
    }
    const std::uint64_t part_bytes = 16ULL * threads * vectors_per_thread;
    if (page_bytes == 0 || page_bytes % part_bytes != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth page probe: page_bytes must be a positive multiple of %llu",
                    static_cast<unsigned long long>(part_bytes));
    }
    if (!key_cache || !value_cache || !sink || (num_pages != 0 && !pages)) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth page probe: null pointer");
    }
    if ((reinterpret_cast<std::uintptr_t>(key_cache) | reinterpret_cast<std::uintptr_t>(value_cache) |
         reinterpret_cast<std::uintptr_t>(sink)) % 16 != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bandwidth page probe: buffers must be 16-byte aligned");
    }
    if (num_pages == 0) return KVFLUX_OK;
    const std::uint64_t parts = page_bytes / part_bytes;
    if (num_pages * parts > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "bandwidth page probe: grid too large");
    const std::uint64_t page_vectors = page_bytes / 16;
    const hipStream_t s = as_stream(stream);
    switch (threads) {
    case 256:
        return probe_pages_vpt<256>(key_cache, value_cache, num_blocks, page_vectors, pages, num_pages,
                                    vectors_per_thread, nontemporal, sink, s);
    case 512:
        return probe_pages_vpt<512>(key_cache, value_cache, num_blocks, page_vectors, pages, num_pages,
                                    vectors_per_thread, nontemporal, sink, s);
    default:
        return probe_pages_vpt<1024>(key_cache, value_cache, num_blocks, page_vectors, pages, num_pages,
                                     vectors_per_thread, nontemporal, sink, s);
    }
}
