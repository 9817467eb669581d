#pragma once
// Owner of physical page ids for the paged KV cache (metadata only; it holds
// no device memory). Same surface as the reference's
// include/kvflux/physical_block_pool.h:22-58. Page state lives in a
// detail::PageLedger, the same ledger BlockManager uses.

#include "kvflux/block_manager.h"

#include <cstddef>

namespace kvflux {

// Index of a page inside PagedKVStorage. Not a pointer and not ownership.
using PhysicalBlockID = std::size_t;
using PhysicalBlockHandle = BlockHandle;

class PhysicalBlockPool {
public:
    PhysicalBlockPool(std::size_t capacity, std::size_t block_size,
                      BlockManager::Hasher hasher = BlockManager::prefix_hash);

    PhysicalBlockPool(const PhysicalBlockPool&) = delete;
    PhysicalBlockPool& operator=(const PhysicalBlockPool&) = delete;
    PhysicalBlockPool(PhysicalBlockPool&&) = delete;
    PhysicalBlockPool& operator=(PhysicalBlockPool&&) = delete;

    // New reference to a free (or evicted idle) page; CapacityError if none.
    PhysicalBlockHandle allocate();
    void retain(PhysicalBlockHandle handle);
    // Drops one reference; the page id becomes reusable after the last one.
    void free(PhysicalBlockHandle handle);

    void publish(PhysicalBlockHandle handle, const Tokens& prefix);
    bool lookup(const Tokens& prefix, PhysicalBlockHandle& out);
    bool is_published(PhysicalBlockHandle handle) const;

    // Page id of a live handle; std::invalid_argument for stale handles.
    PhysicalBlockID id(PhysicalBlockHandle handle) const;
    // id() of n handles at once (same checks and exceptions), into out[0..n).
    // No counterpart in the reference.
    void ids(const PhysicalBlockHandle* handles, std::size_t n, PhysicalBlockID* out) const;
    std::size_t ref_count(PhysicalBlockHandle handle) const;
    std::size_t capacity() const noexcept;
    std::size_t block_size() const noexcept;
    // Free pages plus evictable zero-reference published pages.
    std::size_t available() const noexcept;

private:
    detail::PageLedger ledger_;
};

} // namespace kvflux
