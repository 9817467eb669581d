// Library-internal helpers of the C++ layer: status -> exception mapping,
// device guard, pointer checks and the per-storage metadata scratch. All GPU
// access goes through the C ABI of kvflux_hip.h.
#pragma once

#include "kvflux/v2/paged_kv_storage.h"
#include "kvflux_hip.h"

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace kvflux::v2::detail {

// Throws the exception type the reference uses for each failure class.
inline void check(int status, const char* operation) {
    if (status == KVFLUX_OK) return;
    std::string message = std::string(operation) + ": " + kvflux_last_error();
    switch (status) {
    case KVFLUX_ERR_INVALID_ARGUMENT: throw std::invalid_argument(message);
    case KVFLUX_ERR_OUT_OF_RANGE: throw std::out_of_range(message);
    case KVFLUX_ERR_OVERFLOW: throw std::overflow_error(message);
    default: throw std::runtime_error(message);
    }
}

inline std::size_t mul_checked(std::size_t a, std::size_t b, const char* what) {
    if (b != 0 && a > std::numeric_limits<std::size_t>::max() / b) throw std::overflow_error(what);
    return a * b;
}

// Makes `device` current for the scope and restores the caller's device
// (reference src/v2/paged_kv_write.cu:28-37).
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        check(kvflux_get_device(&previous_), "get device");
        if (previous_ != device) check(kvflux_set_device(device), "set device");
    }
    ~DeviceGuard() noexcept { (void)kvflux_set_device(previous_); }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int previous_ = 0;
};

// Rejects host, managed and foreign-device pointers
// (reference src/v2/paged_kv_write.cu:52-60).
inline void require_device_pointer(const void* pointer, int device, const char* name) {
    int owner = -1;
    if (kvflux_pointer_device(pointer, &owner) != KVFLUX_OK || owner != device) {
        throw std::invalid_argument(std::string(name) + " must be device memory on storage GPU");
    }
}

inline bool overlaps(const void* a, std::size_t a_bytes, const void* b, std::size_t b_bytes) {
    const auto x = reinterpret_cast<std::uintptr_t>(a);
    const auto y = reinterpret_cast<std::uintptr_t>(b);
    return x <= y ? y - x < a_bytes : x - y < b_bytes;
}

// Grow-only device buffer on one device.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    ~DeviceBuffer() noexcept {
        if (ptr_) (void)kvflux_device_free(ptr_);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    // Current device must be the owning device. A new allocation is
    // zero-filled when `zeroed` (the attention workspace relies on it).
    void* reserve(std::size_t bytes, bool zeroed = false) {
        if (bytes <= bytes_) return ptr_;
        if (ptr_) check(kvflux_device_free(ptr_), "free scratch");
        ptr_ = nullptr;
        bytes_ = 0;
        const std::size_t rounded = (bytes + 4095) & ~std::size_t{4095};
        check(kvflux_device_malloc(&ptr_, rounded), "allocate scratch");
        bytes_ = rounded;
        if (zeroed) check(kvflux_fill_bytes(ptr_, 0, rounded, nullptr), "clear scratch");
        return ptr_;
    }
    std::size_t size() const noexcept { return bytes_; }
    void* data() const noexcept { return ptr_; }

private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

class PinnedBuffer {
public:
    PinnedBuffer() = default;
    ~PinnedBuffer() noexcept {
        if (ptr_) (void)kvflux_host_free_pinned(ptr_);
    }
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    void* reserve(std::size_t bytes) {
        if (bytes <= bytes_) return ptr_;
        if (ptr_) check(kvflux_host_free_pinned(ptr_), "free staging");
        ptr_ = nullptr;
        bytes_ = 0;
        const std::size_t rounded = (bytes + 4095) & ~std::size_t{4095};
        check(kvflux_host_malloc_pinned(&ptr_, rounded), "allocate staging");
        bytes_ = rounded;
        return ptr_;
    }

private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

} // namespace kvflux::v2::detail

namespace kvflux::v2::detail {

// Reused across calls of one storage. Every public call synchronises before
// returning, so the buffers are free again when the next call starts.
struct DeviceScratch {
    DeviceBuffer metadata;     // uploaded slot mappings / block tables / lengths
    PinnedBuffer staging;      // host side of those uploads
    DeviceBuffer workspace;    // split-K partials of the attention kernel
    std::vector<std::uint64_t> seen_slots;  // duplicate-slot bitmap (host)

    // Packs host arrays into pinned staging, uploads them with one copy on
    // the default stream and returns their device addresses in order.
    std::vector<const std::uint64_t*> upload(
        const std::vector<std::pair<const void*, std::size_t>>& arrays) {
        std::size_t total = 0;
        std::vector<std::size_t> offsets;
        offsets.reserve(arrays.size());
        for (const auto& [data, bytes] : arrays) {
            offsets.push_back(total);
            total += (bytes + 255) & ~std::size_t{255};
        }
        std::vector<const std::uint64_t*> out(arrays.size(), nullptr);
        if (total == 0) return out;
        auto* host = static_cast<unsigned char*>(staging.reserve(total));
        auto* dev = static_cast<unsigned char*>(metadata.reserve(total));
        for (std::size_t i = 0; i < arrays.size(); ++i) {
            if (arrays[i].second) std::memcpy(host + offsets[i], arrays[i].first, arrays[i].second);
            out[i] = reinterpret_cast<const std::uint64_t*>(dev + offsets[i]);
        }
        check(kvflux_memcpy_async(dev, host, total, nullptr), "upload metadata");
        return out;
    }
};

inline int abi_dtype(DType dtype) {
    switch (dtype) {
    case DType::Float16: return KVFLUX_DTYPE_F16;
    case DType::BFloat16: return KVFLUX_DTYPE_BF16;
    case DType::Float32: return KVFLUX_DTYPE_F32;
    }
    throw std::invalid_argument("unsupported paged KV dtype");
}

// Q and O must be device buffers on the storage GPU, disjoint from each
// other and from the cache.
inline void validate_q_o(const PagedKVStorage& storage, const float* query, float* output,
                         std::size_t tensor_bytes) {
    const auto& layout = storage.layout();
    require_device_pointer(query, storage.device(), "Q");
    require_device_pointer(output, storage.device(), "attention output");
    if (overlaps(query, tensor_bytes, output, tensor_bytes) ||
        overlaps(query, tensor_bytes, storage.key_base(), layout.total_bytes()) ||
        overlaps(output, tensor_bytes, storage.key_base(), layout.total_bytes())) {
        throw std::invalid_argument("Q and attention output must not overlap each other or KV cache");
    }
}

// Split-K workspace of an attention call, grown on demand.
inline void* attention_workspace(const PagedKVStorage& storage, std::size_t rows,
                                 std::size_t kv_len, std::size_t query_heads, std::size_t* bytes) {
    const auto& layout = storage.layout();
    check(kvflux_paged_attention_workspace_size(rows, kv_len, layout.num_kv_heads(), query_heads,
                                                layout.block_size(), layout.head_size(), bytes),
          "attention workspace size");
    return *bytes ? storage.scratch().workspace.reserve(*bytes) : nullptr;
}

// Workspace of the split-key MFMA prefill (nullptr when the call does not split).
inline void* prefill_workspace(const PagedKVStorage& storage, std::size_t query_tokens, std::size_t kv_len,
                               std::size_t query_heads, std::size_t* bytes) {
    const auto& layout = storage.layout();
    check(kvflux_paged_prefill_workspace_size(layout.num_kv_heads(), layout.head_size(), kv_len, query_tokens,
                                              query_heads, bytes),
          "prefill workspace size");
    return *bytes ? storage.scratch().workspace.reserve(*bytes) : nullptr;
}

} // namespace kvflux::v2::detail
