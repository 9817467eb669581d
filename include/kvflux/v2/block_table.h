#pragma once
// Logical -> physical page map of one sequence. Entry i is logical block i.
// Every entry owns one PhysicalBlockPool reference, returned on destruction,
// so the table is move-only. Same surface as the reference's
// include/kvflux/v2/block_table.h:14-61.

#include "kvflux/physical_block_pool.h"

#include <cstddef>
#include <vector>

namespace kvflux::v2 {

class SequenceState;

class BlockTable {
public:
    explicit BlockTable(PhysicalBlockPool& pool) noexcept;
    ~BlockTable() noexcept;

    BlockTable(const BlockTable&) = delete;
    BlockTable& operator=(const BlockTable&) = delete;
    BlockTable(BlockTable&& other) noexcept;
    BlockTable& operator=(BlockTable&& other) noexcept;

    // Allocates a page and appends it; the table is unchanged on failure.
    PhysicalBlockID append_new();
    // Appends `handle` with an extra reference owned by this table.
    void append_existing(PhysicalBlockHandle handle);
    // Shares `source`'s logical block; both tables must use one pool.
    void append_shared(const BlockTable& source, std::size_t logical_block);

    PhysicalBlockID physical_id(std::size_t logical_block) const;
    // physical_id of every entry, in order, into out[0..size()). No
    // counterpart in the reference.
    void physical_ids(PhysicalBlockID* out) const;
    PhysicalBlockHandle handle(std::size_t logical_block) const;
    std::size_t ref_count(std::size_t logical_block) const;
    PhysicalBlockID operator[](std::size_t logical_block) const {
        return physical_id(logical_block);
    }
    std::size_t size() const noexcept { return entries_.size(); }
    bool empty() const noexcept { return entries_.empty(); }
    bool shares_pool_with(const BlockTable& other) const noexcept {
        return pool_ != nullptr && pool_ == other.pool_;
    }
    bool uses_pool(const PhysicalBlockPool& pool) const noexcept { return pool_ == &pool; }
    PhysicalBlockPool& pool() const;

    // Releases the last entry's reference.
    void pop_back();
    // Swaps the last entry for a private, unpublished page whose single
    // reference the caller hands over; the old entry's reference is released.
    void replace_last_owned(PhysicalBlockHandle new_handle);
    void clear() noexcept;

private:
    friend class SequenceState;
    // Makes room for `n` more entries (geometric growth), so that a later
    // adopt() of n handles cannot fail.
    void make_room(std::size_t n);
    // Appends handles whose references the caller hands over; room for them
    // was made first.
    void adopt(const std::vector<PhysicalBlockHandle>& handles) noexcept;

    PhysicalBlockPool* pool_;  // nullptr after being moved from
    std::vector<PhysicalBlockHandle> entries_;
};

} // namespace kvflux::v2
