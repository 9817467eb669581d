#pragma once
// Device memory of a single-layer paged KV cache on one GPU: one allocation
// holding the K region (pool.capacity() pages) followed by the V region.
// Same public surface as the reference's include/kvflux/v2/paged_kv_storage.h:14-45.
// The GPU is reached only through the C ABI in kvflux_hip.h.

#include "kvflux/physical_block_pool.h"
#include "kvflux/v2/paged_kv_layout.h"
#include "kvflux/v2/slot_mapping.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

namespace kvflux::v2 {

namespace detail {
// Per-storage reusable device metadata buffers, pinned staging and the
// split-K workspace; defined in the library.
struct DeviceScratch;
}

class PagedKVStorage {
public:
    PagedKVStorage(PhysicalBlockPool& pool, std::size_t num_kv_heads,
                   std::size_t head_size, DType dtype, int device = 0);
    ~PagedKVStorage();

    PagedKVStorage(const PagedKVStorage&) = delete;
    PagedKVStorage& operator=(const PagedKVStorage&) = delete;

    const PagedKVLayout& layout() const noexcept { return layout_; }
    int device() const noexcept { return device_; }
    bool uses_pool(const BlockTable& table) const noexcept { return table.uses_pool(pool_); }
    void* key_base() const;
    void* value_base() const;

    // Device addresses (not dereferenceable on the host).
    void* page_address(KVKind kind, PhysicalBlockHandle handle) const;
    void* element_address(KVKind kind, PhysicalBlockHandle handle,
                          std::size_t head, std::size_t token, std::size_t dimension) const;
    void* slot_address(KVKind kind, PhysicalSlot slot,
                       std::size_t head, std::size_t dimension) const;

    // Copies the whole K and V page of `source` to the private, unpublished
    // page `destination`, then waits for the copy.
    void copy_block(PhysicalBlockHandle source, PhysicalBlockHandle destination) const;
    // Batch form (no counterpart in the reference): every (source,
    // destination) pair in one kernel launch, then one wait. Destinations
    // must be distinct private, unpublished pages, none of them a source.
    void copy_blocks(
        const std::vector<std::pair<PhysicalBlockHandle, PhysicalBlockHandle>>& pairs) const;

    // Library-internal: reusable device buffers for per-call metadata.
    detail::DeviceScratch& scratch() const { return *scratch_; }

private:
    PhysicalBlockPool& pool_;
    PagedKVLayout layout_;
    int device_;
    void* arena_ = nullptr;
    std::unique_ptr<detail::DeviceScratch> scratch_;
};

} // namespace kvflux::v2
