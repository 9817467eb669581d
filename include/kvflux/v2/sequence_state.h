#pragma once
// Logical KV address space of one request: token count plus BlockTable.
// Same surface as the reference's include/kvflux/v2/sequence_state.h:14-71.

#include "kvflux/v2/block_table.h"

#include <cstddef>
#include <cstdint>
#include <functional>

namespace kvflux::v2 {

using RequestID = std::uint64_t;
class PrefixCache;
namespace detail {
struct SequenceAccess;  // batched appends of the library (copy_on_write.h, device_batch_table.h)
}

struct TokenLocation {
    PhysicalBlockID physical_block;
    std::size_t offset_in_block;
};

class SequenceState {
public:
    SequenceState(RequestID request_id, PhysicalBlockPool& pool) noexcept;

    SequenceState(const SequenceState&) = delete;
    SequenceState& operator=(const SequenceState&) = delete;
    SequenceState(SequenceState&& other) noexcept;
    SequenceState& operator=(SequenceState&& other) noexcept;

    RequestID request_id() const noexcept { return id_; }
    std::size_t num_tokens() const noexcept { return tokens_; }
    std::size_t block_size() const noexcept { return block_size_; }
    const BlockTable& block_table() const noexcept { return table_; }
    std::size_t num_allocated_blocks() const noexcept { return table_.size(); }
    // 0 for an empty request; block_size (not 0) when the tail is full.
    std::size_t last_block_num_tokens() const noexcept;

    // Reserves positions (and pages at block boundaries) for `count` new
    // tokens. All-or-nothing: a failed allocation returns the new pages.
    void append_tokens(std::size_t count);
    TokenLocation append_token();

    // New request sharing every current page, including a partial tail.
    SequenceState fork_shared(RequestID new_request_id) const;

    using BlockCopier = std::function<void(PhysicalBlockHandle source,
                                           PhysicalBlockHandle destination)>;
    // Decode append with copy-on-write of a shared partial tail page.
    TokenLocation append_token_with_copy(const BlockCopier& copy);

    PhysicalBlockID physical_block_id(std::size_t logical_block) const;
    // physical_block_id of every allocated block, in order, into
    // out[0..num_allocated_blocks()). No counterpart in the reference.
    void physical_block_ids(PhysicalBlockID* out) const;
    TokenLocation token_location(std::size_t token_index) const;

private:
    friend class PrefixCache;
    friend struct detail::SequenceAccess;
    // Room for `n` more table entries (std::bad_alloc is the only failure).
    void reserve_blocks(std::size_t n);
    // Maps whole published blocks onto an empty sequence: `handles` carry one
    // reference each, which the table takes over; room was reserved first.
    void adopt_cached_blocks(const std::vector<PhysicalBlockHandle>& handles) noexcept;
    PhysicalBlockHandle block_handle(std::size_t logical_block) const;
    // The tail page is partially filled and shared with another holder.
    bool tail_shared_and_partial() const;

    RequestID id_;
    std::size_t tokens_ = 0;
    std::size_t block_size_;
    BlockTable table_;
};

} // namespace kvflux::v2
